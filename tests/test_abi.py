"""The C-ABI library: built, current, and exporting every symbol include/kdn.h declares with the
argument list the ctypes binding uses (no GPU needed: loading does not touch a device)."""
import pathlib

import pytest

from _header_sigs import HEADER, header_signatures

PKG = pathlib.Path(__file__).resolve().parent.parent / "kalman-delta-networks_amd"
LIB = PKG / "lit_gpt" / "kdn_ops" / "libkdn_hip.so"


def test_binding_matches_header():
    from lit_gpt.kdn_ops import _lib
    sigs = header_signatures()
    assert set(sigs) == set(_lib._SIGS), set(sigs) ^ set(_lib._SIGS)
    for name, (ret, code) in sigs.items():
        assert _lib._SIGS[name] == code, name
        assert (name in _lib._SIZE_FNS) == (ret == "size_t"), name


def test_library_is_current_and_exports_all_symbols():
    if not LIB.exists():
        pytest.skip("libkdn_hip.so not built (run __graft_entry__.build())")
    newest_src = max(p.stat().st_mtime for p in list((PKG / "csrc").glob("*")) + [HEADER])
    assert LIB.stat().st_mtime >= newest_src, "libkdn_hip.so is older than its sources: rebuild"
    import torch  # noqa: F401  (binds the HIP runtime first)
    from lit_gpt.kdn_ops import _lib
    lib = _lib.load()
    for name in header_signatures():
        assert hasattr(lib, name), name
    assert lib.kdn_mem_chunk_size() == 64
    assert _lib.size("kdn_mem_saved_size", 1, 64, 1, 64, 64) > 0


def test_integration_stub_matches_header():
    """The ctypes stub shown to reference-side maintainers declares every entry point with the
    header's argument and return types."""
    import re

    from _header_sigs import header_signatures
    sigs = header_signatures()
    doc = (pathlib.Path(__file__).resolve().parents[1] / "INTEGRATION.md").read_text()
    blk = doc[doc.index("_sig = {"):doc.index("for _n, (_a, _r)")]
    code = {"P": "p", "I": "i", "L": "l", "F": "f", "Z": "z", "S": "s"}
    stub = {}
    for name, args, ret in re.findall(r'"(kdn_\w+)": \(\[([^\]]*)\], (\w)\)', blk, re.S):
        stub[name] = ({"I": "int", "Z": "size_t"}[ret],
                      "".join(code[a.strip()] for a in args.replace("\n", " ").split(",") if a.strip()))
    assert set(stub) == set(sigs), set(stub) ^ set(sigs)
    for name, sig in sigs.items():
        assert stub[name] == tuple(sig), name
