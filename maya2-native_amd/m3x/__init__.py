"""m3x: the Maya3 per-frame decode step on MI355X (gfx950) HIP kernels behind a C ABI (include/m3x.h).

Layout: csrc/ (kernels + C ABI, built into m3x/libm3x.so), m3x/_lib.py (ctypes binding), m3x/ops.py (tensor
wrappers), m3x/serve/ (drop-in surfaces of the reference's serve/ modules), m3x/cb0.py (codebook-0 step),
m3x/frame.py (whole frame in one hipGraph), m3x/synth.py (seeded synthetic workloads), m3x/roofline.py.
"""
__version__ = "0.1.0"
