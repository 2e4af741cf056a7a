"""Writes the golden fixtures under tests/golden/ from the reference's own CPU code.

Runs in the build container only (it needs oracle/_ref/libfrref.so, which `make -C oracle ref`
compiles from the reference's quant/q2_0 and core sources). The fixtures are data: seeded inputs
(or the parameters of this build's own generator, for the large ones) and the reference's outputs.

    python tests/golden/make_golden.py

What each fixture pins (reference file:line of the function that produced the outputs):
  q2_format.npz  repack (quant/q2_0/q2_0.cpp:21-62), quantize_q8 (q2_0.cpp:93-117),
                 matvec_ref (q2_0.cpp:119-140), matvec_avx512 (quant/q2_0/q2_0_avx512.cpp:23-52),
                 dot_ggml (tests/test_q2_0.cpp:44-53 semantics, exported by the shim)
  expert.npz     expert_ffn, both kernels (q2_0.cpp:164-185), config shape n 2048, ff 512
  moe_cpu.npz    moe_cpu (quant/q2_0/moe_cpu.cpp:36-114) over a Miss list, small and config shapes
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

GGML = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])   # ggml block_q2_0: fp16 d, 16 code bytes (18 B)


def random_blocks(rng, rows: int, cols: int) -> np.ndarray:
    """ggml blocks as tests/test_q2_0.cpp:28-37 draws them: d = fp16(|N(0, 0.01)| + 1e-4), uniform bytes."""
    b = np.zeros(rows * (cols // 64), GGML)
    d = (np.abs(rng.normal(0.0, 0.01, b.size)) + 1e-4).astype(np.float32)
    b["d"] = d.astype(np.float16).view(np.uint16)
    b["qs"] = rng.integers(0, 256, (b.size, 16), dtype=np.uint8)
    return b


def q8_inputs(rng) -> np.ndarray:
    """Activation rows with the edge cases of Q8_0: an all-zero block, exact .5 ties after scaling
    (amax 127 gives d = 1), negative ties, a tiny block (subnormal fp16 scale), and normals."""
    x = rng.standard_normal((4, 640)).astype(np.float32)
    x[0, 0:32] = 0.0
    x[0, 32:64] = np.arange(32, dtype=np.float32) - 15.5      # ties at +-.5
    x[0, 63] = 127.0
    x[1, 0:32] = -(np.arange(32, dtype=np.float32) + 0.5)
    x[1, 31] = -127.0
    x[1, 32:64] = rng.standard_normal(32).astype(np.float32) * 1e-6
    x[2, 64:96] = 1e4 * rng.standard_normal(32).astype(np.float32)
    return x


def main() -> None:
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libfrref.so is not built (make -C oracle ref, needs /root/reference)")
    rng = np.random.default_rng(20260927)
    out = {}

    # ---- repack, 8 x 4096 (tests/test_q2_0.cpp:74-86)
    blocks = random_blocks(rng, 8, 4096)
    packed = np.zeros(O.lib().orc_mat_bytes(8, 4096), np.uint8)
    R.ref_repack(blocks.view(np.uint8), 8, 4096, packed)
    out["repack_in"] = blocks.view(np.uint8)
    out["repack_out"] = packed

    # ---- Q8_0
    x = q8_inputs(rng)
    qs = np.zeros(x.size, np.int8)
    d = np.zeros(x.size // 32, np.float32)
    R.ref_quantize_q8(np.ascontiguousarray(x.reshape(-1)), x.size, qs, d)
    out["q8_x"], out["q8_qs"], out["q8_d"] = x, qs.reshape(4, -1), d.reshape(4, -1)

    # ---- matvec at the reference test's shapes, 4 tokens, both kernels; dot_ggml per row
    for rows, cols in ((96, 2560), (160, 640)):
        tag = f"{rows}x{cols}"
        blocks = random_blocks(rng, rows, cols)
        w = np.zeros(O.lib().orc_mat_bytes(rows, cols), np.uint8)
        R.ref_repack(blocks.view(np.uint8), rows, cols, w)
        xs = rng.standard_normal((4, cols)).astype(np.float32)
        yr = np.zeros((4, rows), np.float32)
        R.ref_matvec(w, rows, cols, xs, 4, 0, rows, yr, rows, 0)
        ya = np.zeros((4, 4, rows), np.float32)          # [ntok - 1][t][r]
        for nt in range(1, 5):
            R.ref_matvec(w, rows, cols, np.ascontiguousarray(xs[:nt]), nt, 0, rows, ya[nt - 1], rows, 1)
        dg = np.array([R.ref_dot_ggml(np.ascontiguousarray(blocks[r * (cols // 64):(r + 1) * (cols // 64)]).view(np.uint8),
                                      np.ascontiguousarray(xs[0]), cols) for r in range(rows)], np.float32)
        out[f"mv_{tag}_blocks"] = blocks.view(np.uint8)
        out[f"mv_{tag}_x"] = xs
        out[f"mv_{tag}_ref"] = yr
        out[f"mv_{tag}_avx"] = ya
        out[f"mv_{tag}_dot_ggml"] = dg
    np.savez_compressed(os.path.join(HERE, "q2_format.npz"), **out)

    # ---- one expert at the config shape (blob from this build's generator, cfg 0 layer 0 expert 7)
    n, ff = 2048, 512
    blob = O.gen_expert(0, 0, 7, n, ff)
    xs = rng.standard_normal((4, n)).astype(np.float32)
    ex = {"n": np.int32(n), "ff": np.int32(ff), "gen": np.array([O.SEED, 0, 0, 7], np.int64),
          "blob_sum": np.uint64(int(blob.astype(np.uint64).sum())), "x": xs}
    for use_avx, name in ((0, "ref"), (1, "avx")):
        ys = np.zeros((4, 4, n), np.float32)
        for nt in range(1, 5):
            R.ref_expert_ffn(blob, n, ff, np.ascontiguousarray(xs[:nt]), nt, ys[nt - 1], n, use_avx)
        ex[name] = ys
    np.savez_compressed(os.path.join(HERE, "expert.npz"), **ex)

    # ---- moe_cpu over a Miss list: small shape with ragged token subsets (tests/test_moe_cpu.cpp
    # :17-86 shape), and the decode configuration (T 1, K 10, n 2048, ff 512)
    mc = {}
    pool = R.ref_pool_create(3, 0)
    try:
        for tag, (n, ff, E, T, K) in {"small": (256, 128, 6, 3, 4), "cfg": (2048, 512, 16, 1, 10)}.items():
            blobs = [O.gen_expert(98, 0, e, n, ff) for e in range(E)]
            xs = rng.standard_normal((T, n)).astype(np.float32)
            ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(T)]).astype(np.int32)
            wts = rng.uniform(0.01, 1.0, (T, K)).astype(np.float32)
            ex_, nt_, tk_, wv_ = O.miss_list(ids, wts, E)
            ptrs = (C.c_void_p * len(ex_))(*[blobs[int(e)].ctypes.data for e in ex_])
            prep = R.ref_moe_prepare(pool, n, ff, ptrs, nt_, np.ascontiguousarray(tk_.reshape(-1)),
                                     np.ascontiguousarray(wv_.reshape(-1)), len(ex_), np.ascontiguousarray(xs), T)
            y = np.zeros((T, n), np.float32)
            R.ref_moe_run(pool, prep, y, n)
            R.ref_moe_free(prep)
            mc[f"{tag}_shape"] = np.array([n, ff, E, T, K], np.int32)
            mc[f"{tag}_x"], mc[f"{tag}_ids"], mc[f"{tag}_wts"], mc[f"{tag}_out"] = xs, ids, wts, y
    finally:
        R.ref_pool_destroy(pool)
    mc["gen"] = np.array([O.SEED, 98, 0], np.int64)
    np.savez_compressed(os.path.join(HERE, "moe_cpu.npz"), **mc)
    for f in ("q2_format.npz", "expert.npz", "moe_cpu.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
