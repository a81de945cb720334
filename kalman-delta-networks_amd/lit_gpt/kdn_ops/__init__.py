"""KDN scan operators backed by the gfx950 HIP library libkdn_hip.so."""
