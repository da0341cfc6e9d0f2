"""TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference's algorithm that check the HIP kernels:
  dh_oracle.c + mixer.py   float64 C restatement of the mixer arithmetic (gate pre-activations,
                           level scan, ring-buffer decode step) and the integer mask / ring-slot
                           arithmetic;
  torch_eager.py           the reference's eager PyTorch path (parallel forward and eager
                           incremental decoder), restated functionally over a state dict.
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this package; the
product (dispatcher-hybrid-2_amd/) never does, and its fused paths raise rather than fall back to
anything here.

There is no oracle/_ref build: the reference is Python + Triton with no C/C++ sources.
"""
