"""End-to-end examples that drive FP8Linear through prepare_model (reference tfp8/examples)."""
