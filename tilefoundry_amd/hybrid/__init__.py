"""Decode-step kernels of the hybrid models (workloads C4 and C5): MoE routers
and experts, gated-DeltaNet and Mamba2 recurrences, the full-attention layers'
GQA decode and the fp8 per-channel skinny GEMM.  The C entries are declared in
include/tf_hybrid.h and bound in ``tilefoundry_amd._lib``; ``bench`` times each
kernel at the workloads' shapes against the HBM roofline."""
