"""CPU oracle for the fxlm training hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, in fp32/fp64 torch CPU math, of what the reference's kernels and
wrappers compute (berattunca21-byte/radeon-igpu-forge, ml/fxlm and ml/fxgpu).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only as the checker (or, for the baseline, as the thing timed on the
host CPU).  The product (radeon-igpu-forge_amd/) never imports it.

Modules: attention, cross_entropy, norm, adamw, linear, gpt (the naive-PyTorch
CPU training step that bench.py reports as the CPU baseline).
"""
