"""Shared test helpers: one MoE layer's synthetic weights on the GPU and the same bytes on the host
for the CPU oracle, plus the tolerances the parity tests use.

Tolerances (from the north star in BASELINE.json):
  expert ids and the dispatch permutation: bit-exact;
  routing weights: relative error <= 1e-6;
  layer outputs: per token, max_i |gpu_i - ref_i| / max_i |ref_i| <= 2e-3 (fp32 accumulation).
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

W_REL = 1e-6
OUT_REL = 2e-3

# BASELINE.json configuration shapes
N, FF, E, K = 2048, 512, 512, 10
# Zipf prior strengths of configs 2 and 3 (s) and config 3's alpha, chosen so that a 2048-token
# chunk gives per-expert counts from 0 up to a few hundred
ZIPF_S_STACK, ZIPF_S_PREFILL, PREFILL_ALPHA = 1.1, 1.2, 0.4


def out_rel(gpu: np.ndarray, ref: np.ndarray) -> float:
    gpu = gpu.reshape(ref.shape[0], -1).astype(np.float64)
    ref = ref.reshape(ref.shape[0], -1).astype(np.float64)
    den = np.abs(ref).max(axis=1)
    return float((np.abs(gpu - ref).max(axis=1) / np.maximum(den, 1e-30)).max())


def w_rel(gpu: np.ndarray, ref: np.ndarray) -> float:
    return float((np.abs(gpu.astype(np.float64) - ref) / np.abs(ref.astype(np.float64))).max())


class World:
    """Layer `layer` of BASELINE config `cfg` (n, ff, E, K as given): expert arena, shared expert,
    router and gate weights generated on the GPU by flashrt_amd.gen, and host copies."""

    def __init__(self, cfg: int, layer: int = 0, n: int = N, ff: int = FF, E: int = E, K: int = K,
                 bias: np.ndarray | None = None, norm_input: bool = False):
        import torch
        import flashrt_amd as F
        self.cfg, self.layer, self.n, self.ff, self.E, self.K = cfg, layer, n, ff, E, K
        self.norm_input = norm_input
        self.eb = F.expert_bytes(n, ff)
        self.stride = (self.eb + 4095) // 4096 * 4096
        g = F.gen
        self.arena = torch.empty(E * self.stride, dtype=torch.uint8, device="cuda")
        g.experts(self.arena, self.stride, cfg, layer, 0, E, n, ff)
        self.shared = torch.empty(self.eb, dtype=torch.uint8, device="cuda")
        g.experts(self.shared, self.eb, cfg, layer, 0, 1, n, ff, tensor_base=g.SHARED_TENSOR)
        self.router_w = torch.empty(E * n, dtype=torch.float32, device="cuda")
        g.normal(self.router_w, cfg, layer, g.ROUTER_TENSOR, 0.02)
        self.gate_w = torch.empty(n, dtype=torch.float32, device="cuda")
        g.normal(self.gate_w, cfg, layer, g.GATE_TENSOR, 0.02)
        self.bias_h = bias
        self.bias = None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).cuda()
        torch.cuda.synchronize()
        self.arena_h = self.arena.cpu().numpy()
        self.shared_h = self.shared.cpu().numpy()
        self.router_h = self.router_w.cpu().numpy().reshape(E, n)
        self.gate_h = self.gate_w.cpu().numpy()
        self.layer_obj = F.MoeLayer(self.arena.data_ptr(), self.stride, E, self.shared.data_ptr(), self.router_w,
                                    self.gate_w, n, ff, K, router_bias=self.bias, norm_input=norm_input)

    def blob(self, e: int) -> np.ndarray:
        return self.arena_h[e * self.stride: e * self.stride + self.eb]

    def gpu_forward(self, x: np.ndarray, resid: np.ndarray | None = None):
        import torch
        T = x.shape[0]
        xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
        out = torch.full((T, self.n), float("nan"), dtype=torch.float32, device="cuda")
        ids = torch.full((T, self.K), -1, dtype=torch.int32, device="cuda")
        wts = torch.zeros((T, self.K), dtype=torch.float32, device="cuda")
        r = None if resid is None else torch.from_numpy(np.ascontiguousarray(resid, np.float32)).cuda()
        self.layer_obj.forward(xd, out, T=T, resid=r, ids=ids, wts=wts)
        torch.cuda.synchronize()
        return out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()

    def oracle_forward(self, x: np.ndarray, threads: int = 8):
        return O.moe_layer(self.arena_h, self.stride, self.E, self.shared_h, self.router_h, self.bias_h, self.gate_h,
                           self.n, self.ff, self.K, x, threads=threads, norm_input=self.norm_input)


# ---- the shared expert in a dense GGUF type (ggml ids: F32 0, F16 1, Q8_0 8, BF16 30)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


def dense_tensor(gtype: int, rows: int, cols: int, rng: np.random.Generator, sd: float = 0.02) -> np.ndarray:
    """A seeded [rows][cols] weight matrix in ggml's row-major layout of type gtype, as raw bytes."""
    if gtype == GGML_Q8_0:
        nb = rows * cols // 32
        blk = np.zeros((nb, 34), np.uint8)
        d = (rng.uniform(0.5, 1.5, nb) * sd * 1.7 / 127).astype(np.float16)
        blk[:, :2] = d.view(np.uint8).reshape(nb, 2)
        blk[:, 2:] = rng.integers(-127, 128, (nb, 32)).astype(np.int8).view(np.uint8)
        return blk.reshape(-1)
    w = (rng.standard_normal((rows, cols)) * sd).astype(np.float32)
    if gtype == GGML_F32:
        return w.view(np.uint8).reshape(-1)
    if gtype == GGML_F16:
        return w.astype(np.float16).view(np.uint8).reshape(-1)
    if gtype == GGML_BF16:
        u = w.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)   # round to nearest even
        return r.view(np.uint8).reshape(-1)
    raise ValueError(gtype)


def dense_values(gtype: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The float64 values of a dense ggml matrix (dequantized Q8_0: d * q)."""
    raw = np.ascontiguousarray(raw, np.uint8)
    if gtype == GGML_Q8_0:
        blk = raw.reshape(-1, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
        q = blk[:, 2:].view(np.int8).astype(np.float64)
        return (d * q).reshape(rows, cols)
    if gtype == GGML_F32:
        return raw.view(np.float32).astype(np.float64).reshape(rows, cols)
    if gtype == GGML_F16:
        return raw.view(np.float16).astype(np.float64).reshape(rows, cols)
    if gtype == GGML_BF16:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(rows, cols)
    raise ValueError(gtype)
