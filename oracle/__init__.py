"""CPU oracle of the m3x frame step: TEST INFRASTRUCTURE ONLY.

coracle.py binds the C restatement (m3x_oracle.c) of the bit-exact parts; torch_oracle.py restates the
floating-point parts in PyTorch eager on the CPU. Only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import this package, and only as the reference the GPU results are compared with or as the
timed CPU baseline.
"""
