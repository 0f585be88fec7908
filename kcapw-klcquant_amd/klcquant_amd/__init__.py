"""MI355X (gfx950) implementation of KLCquant's MoE expert path.

Modules:
  mxfp4_expert        — reference-compatible MXFP4 dequant and expert store
  streamed_moe_router — reference-compatible router (top-k, dispatch, experts, combine)
  moe                 — batched MoE layer with every expert resident in HBM
  ops                 — tensor wrappers over the C ABI (include/klc_moe.h)
  synth               — seeded synthetic inputs shared by tests and benchmarks
"""

__all__ = ["mxfp4_expert", "streamed_moe_router", "moe", "ops", "synth"]
