"""CPU oracle of the INT8 kernels — TEST INFRASTRUCTURE ONLY.

Restates the reference's CPU/PyTorch math (dequant -> fp32 attention, the
int8 MLP epilogue order, the quantizers) from scratch.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only
to check or to time the CPU baseline; the shipped library never depends on it.
"""
