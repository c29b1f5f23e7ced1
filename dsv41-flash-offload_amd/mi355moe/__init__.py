"""MI355X-native routed-expert MoE layer (EXL3 3-bpw experts) behind the reference's expert-tier surface.

Modules:
  _lib      ctypes binding of libmi355moe.so (HIP kernels + C ABI, include/mi355moe.h)
  store     HBM-resident expert storage, pointer tables and scale parameters of one layer
  moe       routing prep, decode expert path, fixed-order combine, fixed-shape DecodeRunner
  exl3      the plugin entry points (apply_exl3_fused_moe, apply_exl3_batched_fat) over the store
  ct_vllm   the expert-tier hook surface (install, split/combine entry, slot table, expert cache)
  dma_gemm  the fat-expert staging entry (run_batch)
  workload  seeded synthetic routing and activations of the benchmark configurations
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"
