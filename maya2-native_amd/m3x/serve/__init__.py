"""Drop-in replacements of the reference's serve/ hot-path modules (fast_backbone, fast_depth, fast_depth_kernels,
cache) on the m3x gfx950 kernels."""
