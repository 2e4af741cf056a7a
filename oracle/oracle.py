"""CPU ORACLE — test infrastructure only.

ctypes bindings for oracle/liboracle.so (the clean-room restatement, oracle/moe_oracle.cpp and
oracle/gen.cpp) and, where it was built, oracle/_ref/libfrref.so (the reference's own CPU sources
behind oracle/ref_shim.cpp). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this module; the product path (flashrt_amd) never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libfrref.so")

SEED = 20261201          # master seed of the synthetic inputs
SHARED_TENSOR = 100000   # tensor id of the shared expert in the generator
ROUTER_TENSOR = 3000000  # router weight [E][n]
GATE_TENSOR = 3000001    # shared-expert gate vector [n]
X_TENSOR = 4000000       # activations: X_TENSOR + step

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")

_lib = None
_ref = None


def build() -> None:
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_mat_bytes.restype = C.c_size_t
        L.orc_mat_bytes.argtypes = [C.c_int, C.c_int]
        L.orc_expert_bytes.restype = C.c_size_t
        L.orc_expert_bytes.argtypes = [C.c_int, C.c_int]
        L.orc_repack.argtypes = [_u8p, C.c_int, C.c_int, _u8p]
        L.orc_quantize_q8.argtypes = [_f32p, C.c_int, _i8p, _f32p]
        L.orc_matvec.argtypes = [_u8p, C.c_int, C.c_int, _i8p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int, C.c_int]
        L.orc_expert_ffn.argtypes = [_u8p, C.c_int, C.c_int, _i8p, _f32p, C.c_int, _f32p, C.c_int, C.c_int]
        L.orc_expert_ffn_blk.argtypes = [_u8p, C.c_int, C.c_int, _i8p, _f32p, C.c_int, _f32p, C.c_int, C.c_int, C.c_int]
        L.orc_quantize_q8_blk.argtypes = [_f32p, C.c_int, C.c_int, _i8p, _f32p]
        L.orc_router_logits.argtypes = [_f32p, C.c_int, _f32p, C.c_void_p, C.c_int, C.c_int, _f32p]
        L.orc_dot_canon.restype = C.c_float
        L.orc_dot_canon.argtypes = [_f32p, _f32p, C.c_int]
        L.orc_route_topk.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, _i32p, _f32p, C.c_void_p]
        L.orc_dispatch.argtypes = [_i32p, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p]
        L.orc_moe_cpu.argtypes = [C.c_int, C.c_int, C.c_void_p, _i32p, _i32p, _f32p, C.c_int, _i8p, _f32p, C.c_int,
                                  _f32p, C.c_int, C.c_int, C.c_int]
        L.orc_moe_layer.argtypes = [C.c_void_p, C.c_size_t, C.c_int, _u8p, _f32p, C.c_void_p, _f32p, C.c_int, C.c_int,
                                    C.c_int, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _i32p, _f32p, C.c_void_p, C.c_int]
        L.orc_rmsnorm.argtypes = [_f32p, C.c_int, C.c_int, _f32p]
        L.orc_dense_mv.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_int, _f32p, C.c_int, _f32p]
        L.orc_shexp_ffn.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, _f32p, C.c_int,
                                    _f32p]
        L.orc_moe_layer_shexp.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_int, C.c_void_p, _f32p, C.c_void_p, _f32p, C.c_int, C.c_int,
                                          C.c_int, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _i32p, _f32p, C.c_void_p,
                                          C.c_int]
        L.orc_gen_key.restype = C.c_uint64
        L.orc_gen_key.argtypes = [C.c_uint64] * 4
        L.orc_gen_u64.restype = C.c_uint64
        L.orc_gen_u64.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_gen_normal.restype = C.c_float
        L.orc_gen_normal.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_gen_expert.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _u8p]
        L.orc_gen_normal_f32.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_float, _f32p, C.c_size_t]
        L.orc_gen_zipf_bias.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, _f32p]
        _lib = L
    return _lib


def have_ref() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's compiled CPU path (oracle/_ref), or None when it was not built."""
    global _ref
    if _ref is None and have_ref():
        R = C.CDLL(REF_PATH)
        R.ref_have_avx512.restype = C.c_int
        R.ref_f32_to_f16.restype = C.c_uint16
        R.ref_f32_to_f16.argtypes = [C.c_float]
        R.ref_f16_to_f32.restype = C.c_float
        R.ref_f16_to_f32.argtypes = [C.c_uint16]
        R.ref_expert_bytes.restype = C.c_size_t
        R.ref_expert_bytes.argtypes = [C.c_int, C.c_int]
        R.ref_repack.argtypes = [_u8p, C.c_int, C.c_int, _u8p]
        R.ref_quantize_q8.argtypes = [_f32p, C.c_int, _i8p, _f32p]
        R.ref_matvec.argtypes = [_u8p, C.c_int, C.c_int, _f32p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int, C.c_int]
        R.ref_dot_ggml.restype = C.c_float
        R.ref_dot_ggml.argtypes = [_u8p, _f32p, C.c_int]
        R.ref_expert_ffn.argtypes = [_u8p, C.c_int, C.c_int, _f32p, C.c_int, _f32p, C.c_int, C.c_int]
        R.ref_pool_create.restype = C.c_void_p
        R.ref_pool_create.argtypes = [C.c_int, C.c_int]
        R.ref_pool_create_cpus.restype = C.c_void_p
        R.ref_pool_create_cpus.argtypes = [C.c_int, C.c_void_p, C.c_int]
        R.ref_pool_destroy.argtypes = [C.c_void_p]
        R.ref_physical_cpus.restype = C.c_int
        R.ref_moe_prepare.restype = C.c_void_p
        R.ref_moe_prepare.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, _i32p, _i32p, _f32p, C.c_int, _f32p,
                                      C.c_int]
        R.ref_moe_run.argtypes = [C.c_void_p, C.c_void_p, _f32p, C.c_int]
        R.ref_moe_free.argtypes = [C.c_void_p]
        _ref = R
    return _ref


# ---------------------------------------------------------------- numpy-level helpers

def expert_bytes(n: int, ff: int) -> int:
    return int(lib().orc_expert_bytes(n, ff))


def gen_expert(cfg: int, layer: int, expert: int, n: int, ff: int, sd: float = 0.02, seed: int = SEED) -> np.ndarray:
    blob = np.zeros(expert_bytes(n, ff), np.uint8)
    lib().orc_gen_expert(seed, cfg, layer, expert, n, ff, sd, blob)
    return blob


def gen_normal(cfg: int, layer: int, tensor: int, count: int, sd: float = 1.0, seed: int = SEED) -> np.ndarray:
    out = np.zeros(count, np.float32)
    lib().orc_gen_normal_f32(seed, cfg, layer, tensor, sd, out, count)
    return out


def gen_zipf_bias(cfg: int, layer: int, E: int, s: float, alpha: float = 1.0, seed: int = SEED) -> np.ndarray:
    out = np.zeros(E, np.float32)
    lib().orc_gen_zipf_bias(seed, cfg, layer, E, s, alpha, out)
    return out


def quantize_q8(x: np.ndarray, blk: int = 32):
    """Q8 codes and scales (one per 32 values; a 64-block's scale repeated when blk = 64)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    qs = np.zeros(x.size, np.int8)
    d = np.zeros(x.size // 32, np.float32)
    if blk == 32:
        lib().orc_quantize_q8(x, x.size, qs, d)
    else:
        lib().orc_quantize_q8_blk(x, x.size, blk, qs, d)
    return qs, d


def matvec(w: np.ndarray, rows: int, cols: int, x: np.ndarray, order: int = 0, r0: int = 0, r1: int | None = None):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    nt = x.shape[0]
    r1 = rows if r1 is None else r1
    qs, d = quantize_q8(x)
    y = np.zeros((nt, rows), np.float32)
    lib().orc_matvec(w, rows, cols, qs, d, nt, r0, r1, y, rows, order)
    return y


def expert_ffn(blob: np.ndarray, n: int, ff: int, x: np.ndarray, order: int = 0, blk: int = 32) -> np.ndarray:
    """blk = 64: x and h in Q8 blocks of 64 (moe_q2::run's block64)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, n)
    out = np.zeros_like(x)
    for t0 in range(0, x.shape[0], 4):
        xs = np.ascontiguousarray(x[t0:t0 + 4])
        qs, d = quantize_q8(xs, blk)
        o = np.zeros_like(xs)
        lib().orc_expert_ffn_blk(blob, n, ff, qs, d, xs.shape[0], o, n, order, blk)
        out[t0:t0 + 4] = o
    return out


def router_logits(x: np.ndarray, W: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    E, n = W.shape
    T = x.size // n
    out = np.zeros((T, E), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_router_logits(x.reshape(-1), T, W.reshape(-1), None if b is None else b.ctypes.data, E, n, out)
    return out


def dot_canon(w: np.ndarray, x: np.ndarray) -> float:
    return float(lib().orc_dot_canon(np.ascontiguousarray(w, np.float32), np.ascontiguousarray(x, np.float32), w.size))


def route_topk(logits: np.ndarray, K: int):
    lg = np.ascontiguousarray(logits, np.float32)
    T, E = lg.shape
    ids = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float32)
    counts = np.zeros(E, np.uint32)
    lib().orc_route_topk(lg, T, E, K, ids, w, counts.ctypes.data)
    return ids, w, counts


def dispatch(ids: np.ndarray, E: int):
    ids = np.ascontiguousarray(ids, np.int32)
    T, K = ids.shape
    bounds = np.zeros(E + 1, np.int32)
    tok_of = np.zeros(T * K, np.int32)
    slot_of = np.zeros(T * K, np.int32)
    lib().orc_dispatch(ids.reshape(-1), T, K, E, bounds, tok_of, slot_of)
    return bounds, tok_of, slot_of


def miss_list(ids: np.ndarray, wts: np.ndarray, E: int):
    """moe_block's grouping (moe_ref.cu:166-183): per expert ascending, its tokens in token order,
    at most 4 per Miss. Returns (experts, ntok, tok [m][4], w [m][4])."""
    T, K = ids.shape
    routed = [[] for _ in range(E)]
    for t in range(T):
        for k in range(K):
            routed[int(ids[t, k])].append((t, float(wts[t, k])))
    ex, nt, tk, wv = [], [], [], []
    for e in range(E):
        r = routed[e]
        for i in range(0, len(r), 4):
            c = r[i:i + 4]
            ex.append(e)
            nt.append(len(c))
            tk.append([p[0] for p in c] + [0] * (4 - len(c)))
            wv.append([p[1] for p in c] + [0.0] * (4 - len(c)))
    return (np.array(ex, np.int32), np.array(nt, np.int32), np.array(tk, np.int32).reshape(-1, 4),
            np.array(wv, np.float32).reshape(-1, 4))


def rmsnorm(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    T, n = x.reshape(-1, x.shape[-1]).shape
    u = np.zeros((T, n), np.float32)
    lib().orc_rmsnorm(x.reshape(-1), T, n, u)
    return u


def moe_layer(arena: np.ndarray, stride: int, E: int, shared, router_w: np.ndarray, router_bias,
              gate_w: np.ndarray, n: int, ff: int, K: int, x: np.ndarray, threads: int = 8, order: int = 0,
              norm_input: bool = False):
    """The whole layer (moe_block semantics). arena: uint8 [E*stride] (or an object exposing
    .ctypes.data). shared: the Q2_0 blob, or a tuple (ggml type, gate, up, down, ffs) of the dense
    shared expert (raw ggml-layout bytes). Returns out [T][n], ids, wts, logits."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, n)
    T = x.shape[0]
    out = np.zeros((T, n), np.float32)
    ids = np.zeros((T, K), np.int32)
    wts = np.zeros((T, K), np.float32)
    logits = np.zeros((T, E), np.float32)
    b = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
    if isinstance(shared, tuple):
        st, sg, su, sd, ffs = shared
        sg, su, sd = (np.ascontiguousarray(a).view(np.uint8) for a in (sg, su, sd))
        sp = (st, sg.ctypes.data, su.ctypes.data, sd.ctypes.data, ffs, None)
    else:
        sp = (-1, None, None, None, 0, np.ascontiguousarray(shared, np.uint8).ctypes.data)
    lib().orc_moe_layer_shexp(arena.ctypes.data, stride, E, *sp, np.ascontiguousarray(router_w, np.float32).reshape(-1),
                              None if b is None else b.ctypes.data, np.ascontiguousarray(gate_w, np.float32), n, ff, K,
                              x.reshape(-1), T, threads, order, out, ids, wts, logits.ctypes.data, int(norm_input))
    return out, ids, wts, logits


def dense_mv(gtype: int, w, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """orc_dense_mv: y [T][rows] = W x_t for a ggml-layout dense matrix of type gtype."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    y = np.zeros((x.shape[0], rows), np.float32)
    wb = np.ascontiguousarray(w).view(np.uint8)
    lib().orc_dense_mv(gtype, wb.ctypes.data, rows, cols, x.reshape(-1), x.shape[0], y)
    return y


def shexp_ffn(gtype: int, gate, up, down, n: int, ffs: int, x: np.ndarray) -> np.ndarray:
    """The dense shared expert (orc_shexp_ffn) of ggml type gtype on x [T][n] -> [T][n]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, n)
    out = np.zeros_like(x)
    g, u, d = (np.ascontiguousarray(a).view(np.uint8) for a in (gate, up, down))
    lib().orc_shexp_ffn(gtype, g.ctypes.data, u.ctypes.data, d.ctypes.data, n, ffs, x.reshape(-1), x.shape[0], out)
    return out
