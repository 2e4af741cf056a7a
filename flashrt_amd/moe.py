"""Host-side mirror of the reference's MoE call surface, over the C ABI (include/flashrt_moe.h).

Names, argument order and error behaviour follow the reference's C++ entry points:
  ExpertArena / arena_alloc / arena_free      core/expert_arena.hpp:14-30
  moe_route_topk                              arch/qwen4exp/blocks.hpp:130-135
  moe_q2.workspace_bytes / moe_q2.run         kernels/cuda/moe_q2.h:20-30
  moe_hits_scratch_bytes / moe_hits           arch/qwen4exp/moe_fast.hpp:134-142
  MoeLayer.forward (moe_block_fast / moe_block_stream / moe_block on an HBM arena)
                                              arch/qwen4exp/moe_fast.hpp:144-147, moe_stream.hpp:35,
                                              blocks.hpp:286
Device buffers are torch tensors on the GPU (or raw device addresses as ints); a call enqueues on
the given stream (torch's current stream by default) and raises FrtError where the reference throws
std::runtime_error.
"""
from __future__ import annotations

import ctypes as C
from types import SimpleNamespace

import torch

from ._lib import LAYER_NORM_INPUT, FrtArena, FrtError, FrtExpertSlab, FrtLoadStats, FrtMoeLayer, check, lib

__all__ = ["FrtError", "ExpertArena", "arena_alloc", "arena_free", "moe_route_topk", "router_logits", "quantize_q8",
           "moe_dispatch", "moe_q2", "moe_hits_scratch_bytes", "moe_hits", "MoeLayer", "expert_bytes", "gen",
           "set_option", "layer_sync_error", "MoeStack", "noalloc_scratch_bytes", "q2_repack",
           "q2_repack_expert", "load_experts"]


def _p(t) -> int | None:
    """Device address of a tensor (or an int address, or None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise ValueError("flashrt_amd: expected a device tensor")
    return t.data_ptr()


def _s(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def expert_bytes(d_model: int, d_ff: int) -> int:
    """q2_0::expert_bytes (quant/q2_0/q2_0.hpp:51): gate | up | down planar Q2_0."""
    return int(lib().frt_q2_expert_bytes(d_model, d_ff))


# ---------------------------------------------------------------- arena

class ExpertArena:
    """HBM-resident expert arena: blob(l, e) = base + (l * n_expert + e) * stride, stride a
    multiple of 4 KiB (core/expert_arena.hpp:14-30, on the device instead of host RAM)."""

    def __init__(self, raw: FrtArena):
        self._raw = raw

    @property
    def base(self) -> int:
        return int(self._raw.base)

    @property
    def stride(self) -> int:
        return int(self._raw.stride)

    @property
    def blob_bytes(self) -> int:
        return int(self._raw.blob_bytes)

    @property
    def n_layer(self) -> int:
        return int(self._raw.n_layer)

    @property
    def n_expert(self) -> int:
        return int(self._raw.n_expert)

    def blob(self, layer: int, expert: int) -> int:
        return int(lib().frt_arena_blob(C.byref(self._raw), layer, expert))

    def total_bytes(self) -> int:
        return int(lib().frt_arena_total_bytes(C.byref(self._raw)))

    def upload(self, layer: int, expert: int, host_blob, stream=None) -> None:
        """Copies one host blob (bytes-like / numpy uint8) into (layer, expert)."""
        import numpy as np
        buf = np.ascontiguousarray(np.frombuffer(host_blob, np.uint8) if not isinstance(host_blob, np.ndarray)
                                   else host_blob.view(np.uint8))
        check(lib().frt_arena_upload(C.byref(self._raw), layer, expert, buf.ctypes.data, _s(stream)))
        torch.cuda.current_stream().synchronize() if stream is None else stream.synchronize()

    def free(self) -> None:
        if self._raw.base:
            check(lib().frt_arena_free(C.byref(self._raw)))


def arena_alloc(n_layer: int, n_expert: int, blob_bytes: int) -> ExpertArena:
    raw = FrtArena()
    check(lib().frt_arena_alloc(n_layer, n_expert, blob_bytes, C.byref(raw)))
    return ExpertArena(raw)


def arena_free(a: ExpertArena) -> None:
    a.free()


# ---------------------------------------------------------------- routing and quantization

def moe_route_topk(stream, logits, T: int, E: int, k: int, ids, wts, counts=None, tail_counts=None,
                   tail_from: int = 1 << 30) -> None:
    check(lib().frt_moe_route_topk(_s(stream), _p(logits), T, E, k, _p(ids), _p(wts), _p(counts), _p(tail_counts),
                                   tail_from))


def router_logits(x, T: int, W, E: int, n: int, logits, bias=None, gate_w=None, gate=None, stream=None) -> None:
    check(lib().frt_router_logits(_s(stream), _p(x), T, _p(W), _p(bias), _p(gate_w), E, n, _p(logits), _p(gate)))


def router_logits_gemm(x, T: int, W, E: int, n: int, logits, bias=None, gate_w=None, gate=None, stream=None) -> None:
    """The prefill router (many tokens) as the K-split GEMM on the matrix cores: the same canonical
    order, bit for bit, as router_logits."""
    nb = int(lib().frt_router_gemm_workspace_bytes(T, E, 1 if gate_w is not None else 0))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    check(lib().frt_router_logits_gemm(_s(stream), _p(x), T, _p(W), _p(bias), _p(gate_w), E, n, _p(logits), _p(gate),
                                       _p(ws), nb))


def quantize_q8(x, rows: int, n: int, xq, xd, stream=None) -> None:
    check(lib().frt_quantize_q8(_s(stream), _p(x), rows, n, _p(xq), _p(xd)))


def quantize_pairs(x, rows: int, n: int, block: int, xhi, xlo, stream=None) -> None:
    """frt_quantize_pairs: xhi / xlo [rows][n rounded up to 512] fp16 (the prefill GEMM operand)."""
    check(lib().frt_quantize_pairs(_s(stream), _p(x), rows, n, block, _p(xhi), _p(xlo)))


def moe_dispatch(ids, T: int, K: int, E: int, bounds, tok_of, slot_of, stream=None):
    nbytes = int(lib().frt_moe_dispatch_workspace_bytes(T, K, E))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    check(lib().frt_moe_dispatch(_s(stream), _p(ids), T, K, E, _p(bounds), _p(tok_of), _p(slot_of), _p(ws), nbytes))
    return ws


# ---------------------------------------------------------------- prefill grouped GEMM

def _q2_workspace_bytes(T: int, K: int, n: int, ff: int, E: int) -> int:
    return int(lib().frt_moe_q2_workspace_bytes(T, K, n, ff, E))


def _q2_run(experts, stride: int, E: int, n: int, ff: int, x, ids, T: int, K: int, yd, ws, ws_bytes: int,
            stream=None, block64: bool = False, yd_bf16: bool = False) -> None:
    check(lib().frt_moe_q2_run(_p(experts), stride, E, n, ff, _p(x), _p(ids), T, K, _p(yd), _p(ws), ws_bytes,
                               _s(stream), int(block64), int(yd_bf16)))


moe_q2 = SimpleNamespace(workspace_bytes=_q2_workspace_bytes, run=_q2_run)


# ---------------------------------------------------------------- decode hits

def moe_hits_scratch_bytes(K: int, ff: int, T: int = 1) -> int:
    """moe_hits_scratch_bytes (arch/qwen4exp/moe_fast.hpp:134): the scratch of a moe_hits call of T
    tokens with K slots each, for any n the call takes."""
    return int(lib().frt_moe_hits_scratch_bytes(K, ff, T))


def moe_hits(hit_ptr, hit_n, K: int, x, n: int, ff: int, scratch, yh, stream=None, T: int = 1) -> None:
    check(lib().frt_moe_hits(_p(hit_ptr), _p(hit_n), K, _p(x), n, ff, _p(scratch), _p(yh), _s(stream), T))


# ---------------------------------------------------------------- one layer

class MoeLayer:
    """One MoE layer on the HBM arena: router -> top-k -> routed experts + shared expert *
    sigmoid(gate). T <= 4 runs the decode GEMV path, larger T the grouped MFMA path. norm_input:
    the layer's input is x / rms(x) (the stack's pre-MoE RMS norm)."""

    def __init__(self, experts: int, stride: int, n_expert: int, shared: int, router_w, gate_w, d_model: int,
                 d_ff: int, top_k: int, router_bias=None, norm_input: bool = False):
        self._keep = (router_w, gate_w, router_bias)
        self.raw = FrtMoeLayer(experts, stride, n_expert, shared, _p(router_w), _p(router_bias), _p(gate_w),
                               d_model, d_ff, top_k, LAYER_NORM_INPUT if norm_input else 0)
        self.d_model, self.top_k, self.n_expert = d_model, top_k, n_expert
        self._ws = None

    def set_shared_dense(self, gguf_type: int, gate, up, down, shared_ff: int) -> None:
        """The shared expert as the model's dense GGUF tensors (raw ggml-layout bytes on the device:
        gate / up [shared_ff][d_model], down [d_model][shared_ff]) of type F32, F16, BF16 or Q8_0, in
        place of the Q2_0 blob (frt_moe_layer.shared_dense)."""
        self._shexp = (gate, up, down)
        self.raw.shared_dense = 1
        self.raw.shared_type = int(gguf_type)
        self.raw.shared_ff = int(shared_ff)
        self.raw.shared_gate, self.raw.shared_up, self.raw.shared_down = _p(gate), _p(up), _p(down)
        self._ws = None

    def set_next_router(self, router_w) -> None:
        """The router matrix the next layer call reads; decode calls warm it into the caches
        during their last kernel (frt_moe_layer.next_router_w)."""
        self._next = router_w
        self.raw.next_router_w = _p(router_w)

    def workspace_bytes(self, T: int) -> int:
        return int(lib().frt_moe_layer_workspace_bytes(C.byref(self.raw), T))

    def workspace(self, T: int) -> torch.Tensor:
        need = self.workspace_bytes(T)
        if self._ws is None or self._ws.numel() < need:
            # zeroed: a new allocation may reuse an address the library has seen, with leftover bytes
            self._ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        return self._ws

    def forward(self, x, out, T: int | None = None, resid=None, ids=None, wts=None, counts=None, ws=None,
                stream=None, tail_counts=None, tail_from: int = 1 << 30, probs=None) -> None:
        T = x.shape[0] if T is None else T
        ws = self.workspace(T) if ws is None else ws
        if tail_counts is None and probs is None:
            check(lib().frt_moe_layer_forward(C.byref(self.raw), _p(x), T, _p(resid), _p(out), _p(ids), _p(wts),
                                              _p(counts), _p(ws), ws.numel(), _s(stream)))
        else:
            check(lib().frt_moe_layer_forward_ex(C.byref(self.raw), _p(x), T, _p(resid), _p(out), _p(ids), _p(wts),
                                                 _p(counts), _p(tail_counts), tail_from, _p(probs), _p(ws),
                                                 ws.numel(), _s(stream)))

    def forward_noalloc(self, x, out, T: int | None = None, resid=None, ids=None, wts=None, counts=None,
                        stream=None) -> None:
        """frt_moe_layer_forward_noalloc: a decode window (T <= 4) with the library's static scratch."""
        T = x.shape[0] if T is None else T
        check(lib().frt_moe_layer_forward_noalloc(C.byref(self.raw), _p(x), T, _p(resid), _p(out), _p(ids), _p(wts),
                                                  _p(counts), _s(stream)))


class MoeStack:
    """A stack of single-token MoE layers run as one call (frt_moe_stack_forward):
    x_{l+1} = x_l + moe_l(x_l), out = x_L. All layers share shape, stride and flags."""

    def __init__(self, layers: list):
        self.layers = list(layers)
        self.raw = (FrtMoeLayer * len(self.layers))(*[ml.raw for ml in self.layers])
        self._ws = None

    def refresh(self) -> None:
        """Re-reads the layers' descriptors (after set_next_router on one of them)."""
        for i, ml in enumerate(self.layers):
            self.raw[i] = ml.raw

    def workspace_bytes(self) -> int:
        return int(lib().frt_moe_stack_workspace_bytes(self.raw, len(self.layers)))

    def workspace(self) -> torch.Tensor:
        need = self.workspace_bytes()
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        return self._ws

    def forward(self, x, out, ids=None, wts=None, ws=None, stream=None) -> None:
        ws = self.workspace() if ws is None else ws
        check(lib().frt_moe_stack_forward(self.raw, len(self.layers), _p(x), _p(out), _p(ids), _p(wts), _p(ws),
                                          ws.numel(), _s(stream)))


GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


def router_widen(src: torch.Tensor, gguf_type: int, count: int, dst: torch.Tensor, stream=None) -> None:
    """frt_router_widen: a router or gate tensor in its GGUF type (ggml type id F32, F16, BF16 or
    Q8_0, raw bytes on the device) widened exactly to the fp32 layout the router kernels take."""
    if dst.dtype != torch.float32 or dst.numel() < count:
        raise ValueError("router_widen: dst must be float32 with at least count values")
    check(lib().frt_router_widen(_s(stream), _p(src), int(gguf_type), int(count), _p(dst)))


def set_option(name: str, value: int) -> None:
    """frt_set_option: "decode_fused" (1: single-token layers in one persistent launch, 0: three
    kernels) or "sync_ticks" (bound of the persistent launch's waits, 100 MHz ticks)."""
    check(lib().frt_set_option(name.encode(), int(value)))


def layer_sync_error(ws, stream=None) -> bool:
    """True if a persistent single-token call on this workspace ran out of time since the last check."""
    rc = lib().frt_moe_layer_sync_error(_p(ws), _s(stream))
    if rc < 0:
        check(rc)
    return rc == 1


def noalloc_sync_error(stream=None) -> bool:
    """True if an allocation-free single-token call ran out of time since the last check."""
    rc = lib().frt_noalloc_sync_error(_s(stream))
    if rc < 0:
        check(rc)
    return rc == 1


def q2_repack(ggml_rows, rows: int, cols: int):
    """Planar repack of ggml Q2_0 blocks (host bytes; quant/q2_0/q2_0.cpp:21-62): returns a uint8 array."""
    import numpy as np
    src = np.ascontiguousarray(ggml_rows, dtype=np.uint8)
    out = np.zeros(rows * (cols // 64) * 18, np.uint8)
    nb = lib().frt_q2_repack(src.ctypes.data, rows, cols, out.ctypes.data)
    if nb == 0:
        raise FrtError(-1, lib().frt_last_error().decode())
    return out


def q2_repack_expert(gate, up, down, d_model: int, d_ff: int):
    import numpy as np
    g, u, d = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
    out = np.zeros(expert_bytes(d_model, d_ff), np.uint8)
    check(lib().frt_q2_repack_expert(g.ctypes.data, u.ctypes.data, d.ctypes.data, d_model, d_ff, out.ctypes.data))
    return out


def load_experts(shards: list[str], slabs: list[tuple[int, int]], d_model: int, d_ff: int, arena: ExpertArena,
                 threads: int = 4) -> tuple[float, int]:
    """frt_load_experts: slabs [n_layer * 3] of (shard, file offset) for gate, up, down of each layer.
    Returns (seconds, bytes read)."""
    paths = (C.c_char_p * len(shards))(*[s.encode() for s in shards])
    sl = (FrtExpertSlab * len(slabs))(*[FrtExpertSlab(int(a), int(b)) for a, b in slabs])
    st = FrtLoadStats()
    check(lib().frt_load_experts(C.cast(paths, C.c_void_p), len(shards), C.cast(sl, C.c_void_p), d_model, d_ff,
                                 C.byref(arena._raw), threads, C.byref(st)))
    return st.seconds, int(st.bytes_read)


def noalloc_scratch_bytes() -> int:
    return int(lib().frt_noalloc_scratch_bytes())


# ---------------------------------------------------------------- synthetic inputs

class _Gen:
    SEED = 20261201
    SHARED_TENSOR = 100000
    ROUTER_TENSOR = 3000000
    GATE_TENSOR = 3000001
    X_TENSOR = 4000000

    def experts(self, dst, stride: int, cfg: int, layer: int, e0: int, count: int, n: int, ff: int, sd: float = 0.02,
                tensor_base: int = -1, seed: int | None = None, stream=None) -> None:
        check(lib().frt_gen_experts(self.SEED if seed is None else seed, cfg, layer, e0, count, tensor_base, n, ff, sd,
                                    _p(dst), stride, _s(stream)))

    def normal(self, dst, cfg: int, layer: int, tensor: int, sd: float = 1.0, round_bf16: bool = False,
               seed: int | None = None, stream=None) -> None:
        check(lib().frt_gen_normal(self.SEED if seed is None else seed, cfg, layer, tensor, sd, _p(dst), dst.numel(),
                                   int(round_bf16), _s(stream)))

    def correlated(self, dst, cfg: int, layer: int, tensor0: int, T: int, n: int, rho: float, seed: int | None = None,
                   stream=None) -> None:
        check(lib().frt_gen_correlated(self.SEED if seed is None else seed, cfg, layer, tensor0, T, n, rho, _p(dst),
                                       _s(stream)))

    def zipf_bias(self, cfg: int, layer: int, E: int, s: float, alpha: float = 1.0, seed: int | None = None):
        import numpy as np
        out = np.zeros(E, np.float32)
        lib().frt_gen_zipf_bias(self.SEED if seed is None else seed, cfg, layer, E, s, alpha, out.ctypes.data)
        return out


gen = _Gen()
