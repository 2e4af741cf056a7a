"""flashrt_amd: an MI355X (gfx950) implementation of flashrt's MoE-layer hot path.

The compute is in libflashrt_moe.so (HIP kernels behind the C ABI in include/flashrt_moe.h);
this package is the host-side mirror of the reference's MoE call surface over that library.
"""
from ._lib import FrtError, lib  # noqa: F401
from .moe import (ExpertArena, MoeLayer, arena_alloc, arena_free, expert_bytes, gen, moe_dispatch, moe_hits,  # noqa: F401
                  moe_hits_scratch_bytes, moe_q2, moe_route_topk, quantize_pairs, quantize_q8, router_logits, set_option,
                  layer_sync_error, MoeStack, noalloc_scratch_bytes, noalloc_sync_error, q2_repack, q2_repack_expert,
                  load_experts, router_widen, router_logits_gemm, GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16)

__version__ = "0.1.0"
