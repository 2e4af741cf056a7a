"""CPU tests: the oracle (oracle/liboracle.so, the clean-room restatement of the reference's CPU
path) pinned against the reference's known answers, the golden fixtures written from the
reference's compiled CPU code (tests/golden/make_golden.py), closed forms and brute force.

No GPU is used here. Where oracle/_ref/libfrref.so is built (the build container), the oracle is
also compared with it directly on fresh inputs.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GGML = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def repack(blocks_u8: np.ndarray, rows: int, cols: int) -> np.ndarray:
    w = np.zeros(O.lib().orc_mat_bytes(rows, cols), np.uint8)
    O.lib().orc_repack(np.ascontiguousarray(blocks_u8), rows, cols, w)
    return w


def matvec_q(w, rows, cols, xs, order, r0=0, r1=None, fill=0.0):
    nt = xs.shape[0]
    qs, d = O.quantize_q8(xs)
    y = np.full((nt, rows), fill, np.float32)
    O.lib().orc_matvec(w, rows, cols, qs, d, nt, r0, rows if r1 is None else r1, y, rows, order)
    return y


def dequant_planar(w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Closed form of the planar layout: element j of a 64-block is in byte j % 16 at bits 2 (j / 16),
    and decodes to (code - 1) * d, d the block's fp16 scale stored after all codes."""
    nb = cols // 64
    codes = w[:rows * nb * 16].reshape(rows, nb, 16)
    scales = w[rows * nb * 16:rows * nb * 18].view(np.float16).astype(np.float64).reshape(rows, nb)
    j = np.arange(64)
    q = (codes[:, :, j % 16] >> (2 * (j // 16)).astype(np.uint8)) & 3
    return ((q.astype(np.float64) - 1.0) * scales[:, :, None]).reshape(rows, cols)


def q8_closed_form(x: np.ndarray):
    """ggml quantize_row_q8_0_ref semantics as the reference states them (quant/q2_0/q2_0.cpp:93-117):
    d = amax / 127, stored fp16-rounded; id = 1 / d (unrounded, 0 for d = 0); q = roundf(x * id)."""
    xb = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (xb * idv[:, None]).astype(np.float32)
    q = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))   # half away from zero, as roundf
    return q.astype(np.int8).reshape(x.shape), d.astype(np.float16).astype(np.float32)


# ---------------------------------------------------------------- half precision

def test_fp16_known_answers():
    """tests/test_q2_0.cpp:69-71."""
    L = O.lib()
    assert L.orc_f32_to_f16(1.0) == 0x3C00 and L.orc_f32_to_f16(-2.0) == 0xC000 and L.orc_f32_to_f16(65504.0) == 0x7BFF
    assert L.orc_f16_to_f32(0x3555) == 0.333251953125 and L.orc_f16_to_f32(0x0001) == np.float32(5.960464477539063e-08)


def test_fp16_exhaustive_against_ieee():
    """All 65,536 halves decode as IEEE binary16 (numpy's float16); encoding round-trips every
    finite half and rounds fp32 values to nearest even, subnormals and overflow included."""
    L = O.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    fin = ~nan & np.isfinite(want)
    back = np.array([L.orc_f32_to_f16(float(v)) for v in want[fin]], np.uint16)
    assert np.array_equal(back, h[fin])
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000).astype(np.float32),
                        (np.arange(-2048, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),   # subnormal ties
                        np.float32([65504, 65519.99, 65520, 1e6, -1e6, 0.0, -0.0])])
    got = np.array([L.orc_f32_to_f16(float(v)) for v in f], np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, f.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- Q2_0 layout

def test_sizes():
    """q2_0.hpp:21 mat_bytes and q2_0.cpp:64-80 expert_bytes: 1,382,400 B at 2560/640
    (tests/test_q2_0.cpp:141) and 884,736 B at 2048/512."""
    assert O.lib().orc_mat_bytes(512, 2048) == 294912
    assert O.expert_bytes(2560, 640) == 1382400
    assert O.expert_bytes(2048, 512) == 884736


def test_repack_golden_and_closed_form():
    g = gold("q2_format.npz")
    blocks = g["repack_in"]
    w = repack(blocks, 8, 4096)
    assert np.array_equal(w, g["repack_out"])
    # element-wise placement (tests/test_q2_0.cpp:74-86)
    b = blocks.view(GGML)
    j = np.arange(64)
    ggml_codes = (b["qs"][:, j // 4] >> (2 * (j % 4)).astype(np.uint8)) & 3     # [blocks][64]
    want = np.zeros((b.size, 16), np.uint8)
    for jj in range(64):
        want[:, jj % 16] |= (ggml_codes[:, jj] << (2 * (jj // 16))).astype(np.uint8)
    assert np.array_equal(w[:b.size * 16].reshape(-1, 16), want)
    assert np.array_equal(w[b.size * 16:].view(np.uint16), b["d"])


# ---------------------------------------------------------------- Q8_0

def test_quantize_q8_golden_and_closed_form():
    g = gold("q2_format.npz")
    x = g["q8_x"]
    qs, d = O.quantize_q8(x)
    assert np.array_equal(qs.reshape(4, -1), g["q8_qs"])
    assert np.array_equal(d.reshape(4, -1).view(np.uint32), g["q8_d"].view(np.uint32))
    cq, cd = q8_closed_form(x)
    assert np.array_equal(qs.reshape(x.shape), cq)
    assert np.array_equal(d.reshape(-1), cd)
    assert (qs.reshape(4, -1)[0, :32] == 0).all() and d.reshape(4, -1)[0, 0] == 0.0   # zero block


# ---------------------------------------------------------------- matvec

@pytest.mark.parametrize("rows,cols", [(96, 2560), (160, 640)])
def test_matvec_golden(rows, cols):
    """order 0 == the compiled matvec_ref and == dot_ggml, bit for bit (tests/test_q2_0.cpp:99-109);
    order 1 == the compiled AVX-512 VNNI kernel bit for bit at 1..4 tokens."""
    g = gold("q2_format.npz")
    tag = f"{rows}x{cols}"
    w = repack(g[f"mv_{tag}_blocks"], rows, cols)
    xs = g[f"mv_{tag}_x"]
    y0 = matvec_q(w, rows, cols, xs, 0)
    assert np.array_equal(y0.view(np.uint32), g[f"mv_{tag}_ref"].view(np.uint32))
    assert np.array_equal(y0[0].view(np.uint32), g[f"mv_{tag}_dot_ggml"].view(np.uint32))
    for nt in range(1, 5):
        y1 = matvec_q(w, rows, cols, np.ascontiguousarray(xs[:nt]), 1)
        assert np.array_equal(y1.view(np.uint32), g[f"mv_{tag}_avx"][nt - 1][:nt].view(np.uint32)), nt


def test_matvec_brute_force_and_row_range():
    """Against a float64 dot of the dequantized weights and the Q8 activations (the float order is
    all that may differ), and a row sub-range writes only its rows (tests/test_q2_0.cpp:127-133)."""
    g = gold("q2_format.npz")
    rows, cols = 160, 640
    w = repack(g["mv_160x640_blocks"], rows, cols)
    xs = g["mv_160x640_x"]
    qs, d = O.quantize_q8(xs)
    xa = qs.reshape(4, -1).astype(np.float64) * np.repeat(d.reshape(4, -1), 32, axis=1)
    want = xa @ dequant_planar(w, rows, cols).T
    for order in (0, 1):
        y = matvec_q(w, rows, cols, xs, order)
        assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max(), order
        ys = matvec_q(w, rows, cols, xs[:1], order, 10, 20, fill=-7.0)
        assert ys[0, 9] == -7.0 and ys[0, 20] == -7.0 and np.array_equal(ys[0, 10:20], y[0, 10:20])


# ---------------------------------------------------------------- expert FFN

def test_expert_ffn_golden():
    g = gold("expert.npz")
    n, ff = int(g["n"]), int(g["ff"])
    seed, cfg, layer, e = (int(v) for v in g["gen"])
    blob = O.gen_expert(cfg, layer, e, n, ff, seed=seed)
    assert int(blob.astype(np.uint64).sum()) == int(g["blob_sum"])
    xs = g["x"]
    for order, name in ((0, "ref"), (1, "avx")):
        for nt in range(1, 5):
            qs, d = O.quantize_q8(np.ascontiguousarray(xs[:nt]))
            y = np.zeros((nt, n), np.float32)
            O.lib().orc_expert_ffn(blob, n, ff, qs, d, nt, y, n, order)
            assert np.array_equal(y.view(np.uint32), g[name][nt - 1][:nt].view(np.uint32)), (name, nt)


def test_expert_ffn_vs_float_swiglu():
    """tests/test_q2_0.cpp:156-181: against fp32 SwiGLU on the dequantized weights (no activation
    quantization), relative L2 < 0.05."""
    n, ff = 512, 256
    blob = O.gen_expert(97, 0, 1, n, ff)
    mb = O.lib().orc_mat_bytes(ff, n)
    G = dequant_planar(blob[:mb], ff, n)
    U = dequant_planar(blob[mb:2 * mb], ff, n)
    D = dequant_planar(blob[2 * mb:3 * mb], n, ff)
    x = np.random.default_rng(5).standard_normal((3, n)).astype(np.float32)
    gg, uu = x @ G.T, x @ U.T
    want = (gg / (1 + np.exp(-gg)) * uu) @ D.T
    for order in (0, 1):
        y = O.expert_ffn(blob, n, ff, x, order)
        assert np.linalg.norm(y - want) / np.linalg.norm(want) < 0.05


# ---------------------------------------------------------------- block64 (moe_q2::run's AB = 64)

def q8_closed_form_blk(x: np.ndarray, blk: int):
    """q8_closed_form over blocks of blk values; scales returned one per 32 values."""
    xb = x.reshape(-1, blk).astype(np.float32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (xb * idv[:, None]).astype(np.float32)
    q = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))
    return q.astype(np.int8).reshape(x.shape), np.repeat(d.astype(np.float16).astype(np.float32), blk // 32)


def test_quantize_q8_block64_closed_form():
    """Blocks of 64: one amax, d and id for all 64 values (kernels/cuda/moe_q2.cu:58-81 with AB = 64);
    the scale appears once per 32-value half. blk = 32 is quantize_q8 itself."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(64 * 40) * rng.uniform(0.1, 5, 64 * 40)).astype(np.float32)
    x[64:128] = 0.0                     # a zero block
    x[128:160] = 0.0                    # a block whose first half is zero (d from the second half)
    qs, d = O.quantize_q8(x, 64)
    cq, cd = q8_closed_form_blk(x, 64)
    assert np.array_equal(qs, cq) and np.array_equal(d, cd)
    assert (qs[128:160] == 0).all() and d[4] == d[5] != 0
    q32, d32 = O.quantize_q8(x, 32)
    c32q, c32d = q8_closed_form(x)
    assert np.array_equal(q32, c32q) and np.array_equal(d32, c32d)
    # a 64-block whose two halves share their amax quantizes exactly as two 32-blocks
    y = rng.standard_normal(64 * 8).astype(np.float32)
    y[::32] = 4.0
    assert np.array_equal(O.quantize_q8(y, 64)[0], O.quantize_q8(y, 32)[0])
    assert np.array_equal(O.quantize_q8(y, 64)[1], O.quantize_q8(y, 32)[1])


def test_expert_ffn_block64_composition():
    """expert_ffn with blk = 64 is gate/up matvecs on the 64-block Q8 of x, fp32 SwiGLU, the 64-block
    Q8 of h and the down matvec (composed here from the oracle's matvec on the codes); and against
    fp32 SwiGLU on dequantized weights it stays within the reference test's 0.05 (tests/test_q2_0.cpp:156-181)."""
    n, ff = 640, 384
    blob = O.gen_expert(98, 0, 2, n, ff)
    mb = O.lib().orc_mat_bytes(ff, n)
    x = np.random.default_rng(6).standard_normal((3, n)).astype(np.float32)
    y = O.expert_ffn(blob, n, ff, x, 0, blk=64)

    def mv(w, rows, cols, qs, d):
        out = np.zeros((qs.size // cols, rows), np.float32)
        O.lib().orc_matvec(w, rows, cols, qs, d, qs.size // cols, 0, rows, out, rows, 0)
        return out
    qs, d = O.quantize_q8(x, 64)
    g = mv(blob[:mb], ff, n, qs, d)
    u = mv(blob[mb:2 * mb], ff, n, qs, d)
    h = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
    hq, hd = O.quantize_q8(h, 64)
    want = mv(blob[2 * mb:3 * mb], n, ff, hq, hd)
    assert np.max(np.abs(y - want)) <= 1e-4 * np.max(np.abs(want))   # exp in numpy vs libm: rare code flips
    G = dequant_planar(blob[:mb], ff, n)
    U = dequant_planar(blob[mb:2 * mb], ff, n)
    D = dequant_planar(blob[2 * mb:3 * mb], n, ff)
    gg, uu = x @ G.T, x @ U.T
    ref = (gg / (1 + np.exp(-gg)) * uu) @ D.T
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 0.05
    assert not np.array_equal(y, O.expert_ffn(blob, n, ff, x, 0, blk=32))   # the block size matters


# ---------------------------------------------------------------- moe_cpu

@pytest.mark.parametrize("tag", ["small", "cfg"])
def test_moe_cpu_golden_and_pool_invariance(tag):
    """The compiled moe_cpu output, bit for bit in the VNNI order, for 1, 3 and 6 worker threads
    (tests/test_moe_cpu.cpp:71-86: the pool size does not change the result)."""
    g = gold("moe_cpu.npz")
    n, ff, E, T, K = (int(v) for v in g[f"{tag}_shape"])
    seed, cfg, layer = (int(v) for v in g["gen"])
    blobs = [O.gen_expert(cfg, layer, e, n, ff, seed=seed) for e in range(E)]
    xs, ids, wts = g[f"{tag}_x"], g[f"{tag}_ids"], g[f"{tag}_wts"]
    ex, nt, tk, wv = O.miss_list(ids, wts, E)
    ptrs = (C.c_void_p * len(ex))(*[blobs[int(e)].ctypes.data for e in ex])
    qs, d = O.quantize_q8(xs)
    for threads in (1, 3, 6):
        y = np.zeros((T, n), np.float32)
        O.lib().orc_moe_cpu(n, ff, ptrs, nt, np.ascontiguousarray(tk.reshape(-1)), np.ascontiguousarray(wv.reshape(-1)),
                            len(ex), qs, d, T, y, n, threads, 1)
        assert np.array_equal(y.view(np.uint32), g[f"{tag}_out"].view(np.uint32)), threads
    # and equal, to float rounding, to the sum of per-token expert FFNs it stands for
    want = np.zeros((T, n), np.float64)
    for t in range(T):
        for k in range(K):
            want[t] += wts[t, k] * O.expert_ffn(blobs[int(ids[t, k])], n, ff, xs[t:t + 1], 1)[0]
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()


# ---------------------------------------------------------------- routing

def test_route_topk_reference_recipe():
    """tests/test_route_topk.cpp:22-69: T 16384, E 512, K 10, logits round(N(0, 2) * 4) / 4 (many
    exact ties). ids == a stable sort by logit descending (ties to the lower id); counts exact;
    weights within 1e-6 relative of a float64 softmax renormalised over the selection."""
    T, E, K = 16384, 512, 10
    rng = np.random.default_rng(9)
    lg = (np.round(rng.normal(0.0, 2.0, (T, E)) * 4) / 4).astype(np.float32)
    ids, w, counts = O.route_topk(lg, K)
    want = np.argsort(-lg, axis=1, kind="stable")[:, :K]
    assert np.array_equal(ids, want)
    assert np.array_equal(counts, np.bincount(want.reshape(-1), minlength=E).astype(np.uint32))
    l64 = lg.astype(np.float64)
    p = np.exp(l64 - l64.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    sel = np.take_along_axis(p, want, axis=1)
    ref = sel / sel.sum(axis=1, keepdims=True)
    assert (np.abs(w - ref) / ref).max() <= 1e-6
    assert (np.diff(np.take_along_axis(lg, ids, axis=1), axis=1) <= 0).all()   # monotone selection


def test_route_topk_small_cases():
    # all equal: ids 0..K-1, equal weights; K = E: a full sort
    ids, w, _ = O.route_topk(np.zeros((2, 16), np.float32), 4)
    assert np.array_equal(ids, np.tile(np.arange(4), (2, 1))) and np.allclose(w, 0.25, rtol=0, atol=1e-7)
    lg = np.random.default_rng(3).standard_normal((3, 8)).astype(np.float32)
    ids, w, _ = O.route_topk(lg, 8)
    assert np.array_equal(ids, np.argsort(-lg, axis=1, kind="stable"))
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


@pytest.mark.parametrize("T,K,E", [(1, 10, 512), (3, 10, 512), (2048, 10, 512), (7, 1, 5), (64, 8, 1000)])
def test_dispatch_is_stable_counting_sort(T, K, E):
    """kernels/cuda/moe_q2.cu:83-168: rows are the slots s = t K + k sorted by expert, stable in s."""
    rng = np.random.default_rng(T * 31 + K)
    ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(T)]).astype(np.int32)
    bounds, tok_of, slot_of = O.dispatch(ids, E)
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    assert np.array_equal(slot_of, order) and np.array_equal(tok_of, order // K)
    assert np.array_equal(bounds, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    assert bounds[E] == T * K and np.array_equal(np.sort(slot_of), np.arange(T * K))


# ---------------------------------------------------------------- router logits and RMS norm

def test_router_logits_canonical_order():
    """The canonical order (64 fmaf chains over contiguous runs, adjacent pairwise tree, + bias):
    exact on integer data (no rounding anywhere), within float rounding of a float64 dot otherwise,
    and not symmetric in (T, E) (a transposed operand fails)."""
    rng = np.random.default_rng(4)
    T, E, n = 5, 37, 256
    xi = rng.integers(-8, 9, (T, n)).astype(np.float32)
    Wi = rng.integers(-8, 9, (E, n)).astype(np.float32)
    bi = rng.integers(-4, 5, E).astype(np.float32)
    assert np.array_equal(O.router_logits(xi, Wi, bi), (xi.astype(np.int64) @ Wi.T.astype(np.int64) + bi).astype(np.float32))
    x = rng.standard_normal((T, n)).astype(np.float32)
    W = (rng.standard_normal((E, n)) * 0.02).astype(np.float32)
    got = O.router_logits(x, W)
    want = x.astype(np.float64) @ W.T.astype(np.float64)
    bound = 1e-6 * (np.abs(x).astype(np.float64) @ np.abs(W).T.astype(np.float64))
    assert (np.abs(got - want) <= bound).all()
    # one chain per 64-run: the result depends on the order, and matches dot_canon row by row
    for t in range(T):
        for e in range(0, E, 9):
            assert O.dot_canon(W[e], x[t]) == got[t, e]


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((4, 2048)) * [[1e-3], [1.0], [30.0], [0.0]]).astype(np.float32)
    u = O.rmsnorm(x)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6)
    assert np.abs(u - want).max() <= 2e-6 * np.abs(want).max()
    assert (u[3] == 0).all()


# ---------------------------------------------------------------- synthetic generator

def test_generator_properties():
    a = O.gen_normal(2, 0, 5, 200000)
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    assert np.array_equal(a, O.gen_normal(2, 0, 5, 200000))            # deterministic
    assert not np.array_equal(a[:1000], O.gen_normal(2, 0, 6, 1000))    # independent streams
    assert abs(np.corrcoef(a[:100000], O.gen_normal(2, 1, 5, 100000))[0, 1]) < 0.02
    blob = O.gen_expert(2, 0, 3, 512, 256)
    mb = O.lib().orc_mat_bytes(256, 512)
    codes = blob[:256 * 512 // 4]
    q = np.concatenate([(codes >> s) & 3 for s in (0, 2, 4, 6)])
    assert abs(np.bincount(q, minlength=4) / q.size - 0.25).max() < 0.01
    sc = blob[256 * 512 // 4:mb].view(np.float16).astype(np.float32)
    assert (sc >= 0).all() and 0.01 < sc.mean() < 0.03
    bias = O.gen_zipf_bias(2, 0, 512, 1.1, 0.5)
    want = -1.1 * 0.5 * np.log1p(np.arange(512, dtype=np.float64))
    assert np.allclose(np.sort(bias)[::-1], want, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- the whole layer

def test_moe_layer_composition():
    """orc_moe_layer == its parts: canonical router -> top-k -> per-expert Miss list -> moe_cpu, +
    shared expert * sigmoid(gate), with and without the input RMS norm."""
    n, ff, E, K, T = 256, 128, 12, 3, 5
    rng = np.random.default_rng(8)
    stride = O.expert_bytes(n, ff)
    arena = np.concatenate([O.gen_expert(96, 0, e, n, ff) for e in range(E)])
    shared = O.gen_expert(96, 0, 999, n, ff)
    Wr = (rng.standard_normal((E, n)) * 0.05).astype(np.float32)
    gw = (rng.standard_normal(n) * 0.05).astype(np.float32)
    x = rng.standard_normal((T, n)).astype(np.float32)
    for norm in (False, True):
        out, ids, wts, lg = O.moe_layer(arena, stride, E, shared, Wr, None, gw, n, ff, K, x, threads=2, order=1,
                                        norm_input=norm)
        u = O.rmsnorm(x) if norm else x
        assert np.array_equal(lg, O.router_logits(u, Wr))
        rid, rw, _ = O.route_topk(lg, K)
        assert np.array_equal(ids, rid) and np.array_equal(wts, rw)
        want = np.zeros((T, n), np.float64)
        for t in range(T):
            for k in range(K):
                want[t] += wts[t, k] * O.expert_ffn(arena[ids[t, k] * stride:(ids[t, k] + 1) * stride], n, ff, u[t:t + 1], 1)[0]
            g = 1 / (1 + np.exp(-float(O.dot_canon(gw, u[t]))))
            want[t] += g * O.expert_ffn(shared, n, ff, u[t:t + 1], 1)[0]
        assert np.abs(out - want).max() <= 1e-5 * np.abs(want).max(), norm


# ---------------------------------------------------------------- against the compiled reference, where built

@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (needs /root/reference)")
def test_oracle_vs_compiled_reference_fresh_inputs():
    R = O.ref()
    rng = np.random.default_rng(77)
    for rows, cols in ((64, 2048), (2048, 512)):
        blocks = np.zeros(rows * cols // 64, GGML)
        blocks["d"] = (np.abs(rng.normal(0, 0.01, blocks.size)) + 1e-4).astype(np.float16).view(np.uint16)
        blocks["qs"] = rng.integers(0, 256, (blocks.size, 16), dtype=np.uint8)
        w = repack(blocks.view(np.uint8), rows, cols)
        wr = np.zeros_like(w)
        R.ref_repack(np.ascontiguousarray(blocks.view(np.uint8)), rows, cols, wr)
        assert np.array_equal(w, wr)
        xs = rng.standard_normal((3, cols)).astype(np.float32)
        for use_avx in (0, 1):
            yr = np.zeros((3, rows), np.float32)
            R.ref_matvec(w, rows, cols, xs, 3, 0, rows, yr, rows, use_avx)
            assert np.array_equal(matvec_q(w, rows, cols, xs, use_avx).view(np.uint32), yr.view(np.uint32))


# ---------------------------------------------------------------- the dense shared expert

@pytest.mark.parametrize("gtype", [0, 1, 8, 30])
def test_dense_mv_closed_form(gtype):
    """orc_dense_mv against float64 closed forms: dense types, sum_j w_j x_j on the exact float
    values (within 1e-6 of each row's |w|.|x|); Q8_0, per 32-block the exact integer sum of
    q_w q_a (numpy int64) times d_w d_a, on the oracle's own Q8_0 of x (pinned elsewhere), within
    1e-6 of the row's sum of |terms|. A transposed operand or a dropped block fails both."""
    from tests import helpers as H
    rng = np.random.default_rng(100 + gtype)
    rows, cols, T = 96, 512, 3
    w = H.dense_tensor(gtype, rows, cols, rng)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    y = O.dense_mv(gtype, w, rows, cols, x)
    if gtype == 8:
        blk = w.reshape(rows, cols // 32, 34)
        dw = blk[:, :, :2].copy().view(np.float16).astype(np.float64)[..., 0]
        qw = blk[:, :, 2:].view(np.int8).astype(np.int64)
        for t in range(T):
            qa, da = O.quantize_q8(x[t:t + 1])
            qa = qa.reshape(cols // 32, 32).astype(np.int64)
            sumi = np.einsum("rbj,bj->rb", qw, qa)
            terms = sumi * dw * da.reshape(-1).astype(np.float64)
            want = terms.sum(axis=1)
            assert np.all(np.abs(y[t] - want) <= 1e-6 * np.abs(terms).sum(axis=1) + 1e-30)
    else:
        wv = H.dense_values(gtype, w, rows, cols)
        want = wv @ x.astype(np.float64).T
        bound = np.abs(wv) @ np.abs(x.astype(np.float64)).T
        assert np.all(np.abs(y.T - want) <= 1e-6 * bound)
    # a known answer: unit weights and unit inputs give cols per row (Q8_0: d = 1, q = 1; x = 1
    # quantizes to q = 127 with d = fp16(1/127), so each block sums 32 * 127 * d)
    if gtype == 8:
        blk = np.zeros((rows * cols // 32, 34), np.uint8)
        blk[:, :2] = np.array([np.float16(1.0)]).view(np.uint8)
        blk[:, 2:] = 1
        y1 = O.dense_mv(8, blk.reshape(-1), rows, cols, np.ones((1, cols), np.float32))
        d = float(np.float16(1.0 / 127))
        assert np.allclose(y1, cols / 32 * float(np.float32(4064) * np.float32(d)), rtol=1e-6)


@pytest.mark.parametrize("gtype", [0, 1, 8, 30])
def test_shexp_ffn_composition(gtype):
    """orc_shexp_ffn equals its composition from orc_dense_mv: gate and up products, SwiGLU in
    fp32, then the down product (on h quantized to Q8_0 for the Q8_0 type), within 2e-3 of each
    token's largest output (float rounding of h may move a Q8 code)."""
    from tests import helpers as H
    rng = np.random.default_rng(7 + gtype)
    n, ffs, T = 512, 256, 3
    g, u, d = (H.dense_tensor(gtype, r, c, rng) for r, c in ((ffs, n), (ffs, n), (n, ffs)))
    x = rng.standard_normal((T, n)).astype(np.float32)
    out = O.shexp_ffn(gtype, g, u, d, n, ffs, x)
    gv = O.dense_mv(gtype, g, ffs, n, x)
    uv = O.dense_mv(gtype, u, ffs, n, x)
    h = (gv / (np.float32(1) + np.exp(-gv)) * uv).astype(np.float32)
    want = O.dense_mv(gtype, d, n, ffs, h)
    err = np.abs(out - want).max(axis=1) / np.abs(want).max(axis=1)
    assert err.max() <= 2e-3, err
    assert np.abs(out).max() > 0


def test_moe_layer_with_dense_shared_expert():
    """orc_moe_layer_shexp with a dense (Q8_0) shared expert = the layer with a zero-weight Q2_0
    shared blob (routed part only) plus sigmoid(gate) times orc_shexp_ffn, per token."""
    from tests import helpers as H
    rng = np.random.default_rng(5)
    n, ff, E, K, T = 512, 128, 16, 3, 5
    stride = O.expert_bytes(n, ff)
    arena = np.concatenate([O.gen_expert(0, 0, e, n, ff) for e in range(E)])
    zero_shared = np.zeros(stride, np.uint8)   # all scales 0: the shared term vanishes
    router = (rng.standard_normal((E, n)) * 0.05).astype(np.float32)
    gate = (rng.standard_normal(n) * 0.05).astype(np.float32)
    ffs = 256
    g, u, d = (H.dense_tensor(8, r, c, rng) for r, c in ((ffs, n), (ffs, n), (n, ffs)))
    x = rng.standard_normal((T, n)).astype(np.float32)
    out, ids, wts, lg = O.moe_layer(arena, stride, E, (8, g, u, d, ffs), router, None, gate, n, ff, K, x)
    routed, ids0, wts0, _ = O.moe_layer(arena, stride, E, zero_shared, router, None, gate, n, ff, K, x)
    assert np.array_equal(ids, ids0) and np.array_equal(wts, wts0)
    sh = O.shexp_ffn(8, g, u, d, n, ffs, x)
    gl = np.array([O.lib().orc_dot_canon(gate, np.ascontiguousarray(x[t]), n) for t in range(T)], np.float32)
    sg = (np.float32(1) / (np.float32(1) + np.exp(-gl))).astype(np.float32)
    want = routed + sh * sg[:, None]
    assert np.allclose(out, want, rtol=1e-6, atol=1e-6)
