"""MI355X-native drop-in for the Kalman Delta Network scan path of lit_gpt (kdn_ops)."""
