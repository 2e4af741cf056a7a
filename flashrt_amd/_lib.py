"""Loader for libflashrt_moe.so (the HIP library built from flashrt_amd/csrc).

The product path has no fallback: if the library is missing or fails to load, every entry point
raises. Build it with `make -C flashrt_amd/csrc` (or __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libflashrt_moe.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "flashrt_moe.h")

_vp, _i, _sz, _u64, _f = C.c_void_p, C.c_int, C.c_size_t, C.c_uint64, C.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "frt_last_error": (C.c_char_p, []),
    "frt_version": (C.c_char_p, []),
    "frt_timing_begin": (None, []),
    "frt_timing_end": (_i, [_vp, _i, _vp, _vp, _i]),
    "frt_q2_mat_bytes": (_sz, [_i, _i]),
    "frt_q2_expert_bytes": (_sz, [_i, _i]),
    "frt_arena_alloc": (_i, [_i, _i, _sz, _vp]),
    "frt_arena_free": (_i, [_vp]),
    "frt_arena_blob": (_vp, [_vp, _i, _i]),
    "frt_arena_total_bytes": (_sz, [_vp]),
    "frt_arena_upload": (_i, [_vp, _i, _i, _vp, _vp]),
    "frt_moe_route_topk": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _i]),
    "frt_router_logits": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "frt_quantize_q8": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "frt_quantize_pairs": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp]),
    "frt_router_widen": (_i, [_vp, _vp, _i, _sz, _vp]),
    "frt_router_gemm_workspace_bytes": (_sz, [_i, _i, _i]),
    "frt_router_logits_gemm": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _sz]),
    "frt_moe_dispatch_workspace_bytes": (_sz, [_i, _i, _i]),
    "frt_moe_dispatch": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _sz]),
    "frt_moe_q2_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "frt_moe_q2_run": (_i, [_vp, _sz, _i, _i, _i, _vp, _vp, _i, _i, _vp, _vp, _sz, _vp, _i, _i]),
    "frt_moe_hits_scratch_bytes": (_sz, [_i, _i, _i]),
    "frt_moe_hits": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp, _vp, _vp, _i]),
    "frt_moe_layer_workspace_bytes": (_sz, [_vp, _i]),
    "frt_moe_layer_forward": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "frt_set_option": (_i, [C.c_char_p, C.c_int64]),
    "frt_q2_repack": (_sz, [_vp, _i, _i, _vp]),
    "frt_q2_repack_expert": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "frt_load_experts": (_i, [_vp, _i, _vp, _i, _i, _vp, _i, _vp]),
    "frt_moe_layer_forward_ex": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _sz, _vp]),
    "frt_noalloc_scratch_bytes": (_sz, []),
    "frt_moe_layer_forward_noalloc": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "frt_moe_stack_workspace_bytes": (_sz, [_vp, _i]),
    "frt_moe_stack_forward": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "frt_moe_layer_sync_error": (_i, [_vp, _vp]),
    "frt_noalloc_sync_error": (_i, [_vp]),
    "frt_gen_experts": (_i, [_u64, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "frt_gen_normal": (_i, [_u64, _i, _i, _i, _f, _vp, _sz, _i, _vp]),
    "frt_gen_correlated": (_i, [_u64, _i, _i, _i, _i, _i, _f, _vp, _vp]),
    "frt_gen_zipf_bias": (None, [_u64, _i, _i, _i, _f, _f, _vp]),
}


LAYER_NORM_INPUT = 1


class FrtError(RuntimeError):
    """A C-ABI call returned a nonzero status (the reference throws std::runtime_error)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class FrtArena(C.Structure):
    _fields_ = [("base", C.c_void_p), ("blob_bytes", C.c_size_t), ("stride", C.c_size_t),
                ("n_layer", C.c_int), ("n_expert", C.c_int)]


class FrtMoeLayer(C.Structure):
    _fields_ = [("experts", C.c_void_p), ("stride", C.c_size_t), ("n_expert", C.c_int), ("shared", C.c_void_p),
                ("router_w", C.c_void_p), ("router_bias", C.c_void_p), ("gate_w", C.c_void_p),
                ("d_model", C.c_int), ("d_ff", C.c_int), ("top_k", C.c_int), ("flags", C.c_int),
                ("next_router_w", C.c_void_p), ("shared_dense", C.c_int), ("shared_type", C.c_int),
                ("shared_ff", C.c_int), ("shared_gate", C.c_void_p), ("shared_up", C.c_void_p),
                ("shared_down", C.c_void_p)]


class FrtExpertSlab(C.Structure):
    _fields_ = [("shard", C.c_int), ("file_offset", C.c_uint64)]


class FrtLoadStats(C.Structure):
    _fields_ = [("seconds", C.c_double), ("bytes_read", C.c_uint64)]


_lib = None


def lib():
    """The loaded HIP library; raises if it is not built (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"flashrt_amd: {LIB_PATH} is not built; run `make -C flashrt_amd/csrc`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise FrtError(rc, lib().frt_last_error().decode())
