"""echo-hip: echo-core's decode hot path on MI355X (gfx950).

The product is libechohip.so (C ABI in include/echo_hip.h); this package holds
its ctypes binding (lib), the seeded synthetic-input generator (synth) and the
device-side engine helpers used by bench.py.
"""
