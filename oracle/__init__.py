"""CPU oracle for the tfp8 FP8Linear path -- TEST INFRASTRUCTURE ONLY.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker or
the timed CPU baseline; the product package (fp8-compatibility-layer_amd/tfp8) never imports it.
"""
