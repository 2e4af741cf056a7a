// Router logits, Q8_0 activation quantization and top-k routing.
//
// Router logits use one canonical float order, shared with the CPU oracle, so that expert ids
// match bit for bit: logit[t][e] = the adjacent pairwise tree ((c0+c1)+(c2+c3))+... over 64 chains,
// chain j = fmaf over k in [j L, (j+1) L) ascending from 0 (L = n / 64), then + bias[e]. On the GPU
// a wave owns one router row: lane j is chain j and wave_sum_tree (DPP) is exactly that tree.
//
// Top-k (arch/qwen4exp/moe_ref.cu:21-77 semantics): rank by logit descending, ties to the lower
// expert id; p = exp(l - max) / sum (sum in double); weights p_k / max(sum_k p_k, 2^-14).
#include "common.hpp"
#include "topk.hpp"

namespace frt {
namespace {

constexpr int kMaxE = 1024;   // experts a routing wave handles (16 logits per lane)

// Q8_0 of one 32-value block held by the 32 lanes of a half-wave (lane j has element j): writes
// codes and the fp16-rounded scale (quant/q2_0/q2_0.cpp:93-108).
__device__ __forceinline__ void quant32(float v, int j, int8_t* q, float* d) {
    const float am = half_max(fabsf(v));
    const float dd = q8_scale(am);
    q[j] = int8_t(q8_code(v, q8_inv(dd)));
    if (j == 0) *d = f16_round(dd);
}

// ---- router: grid (ceil(rows / W), ceil(T / tok_per_wg)), W = blockDim.x / 64 waves, one router row
// each (W = 2 for decode windows, so that the 4 MiB of router rows spread over twice as many CUs).
// Rows 0..E-1 are the router (bias optional); row E (when gate_w) is the shared expert's gate.
// x tiles of TT tokens are staged in LDS with each 64-chain padded by one float (conflict-free).
// norm: the layer input is u = x * r, r the canonical RMS scale of the token (topk.hpp); u_i is
// formed as a rounded product before its fma, exactly as the CPU oracle does.
// xq/xd (optional, T <= tok_per_wg): Q8_0 of the experts' input (u when norm, else x), one
// 32-value block per half-wave spread over the workgroups of grid row 0.
template <int L>
__global__ void __launch_bounds__(256) k_router(const float* __restrict__ x, int T, const float* __restrict__ W,
                                                const float* __restrict__ bias, const float* __restrict__ gate_w,
                                                int E, float* __restrict__ logits, float* __restrict__ gate, int TT,
                                                int tok_per_wg, int norm, int8_t* __restrict__ xq,
                                                float* __restrict__ xd) {
    extern __shared__ float xs[];   // [TT][64][L + 1]
    __shared__ float s_r[64];
    const int n = 64 * L;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + wave;
    const bool is_gate = row == E;
    const bool live = row < E || (is_gate && gate_w);
    const float* w = is_gate ? gate_w : W + size_t(row < E ? row : 0) * n;
    float wr[L];
    {   // this lane's chain of the router row: L contiguous floats as L/4 16-byte loads
        // (loaded unconditionally, row 0 standing in for a row that is not live, whose wave skips the
        // dot product: a conditional load would be waited for where the branches meet)
        const float4* w4 = reinterpret_cast<const float4*>(w + lane * L);
#pragma unroll
        for (int i = 0; i < L / 4; ++i) {
            const float4 v = w4[i];
            wr[4 * i] = v.x;
            wr[4 * i + 1] = v.y;
            wr[4 * i + 2] = v.z;
            wr[4 * i + 3] = v.w;
        }
    }
    const float b = bias ? bias[min(row, E - 1)] : 0.0f;   // used for rows < E only
    const int t_begin = blockIdx.y * tok_per_wg, t_end = min(T, t_begin + tok_per_wg);
    for (int t0 = t_begin; t0 < t_end; t0 += TT) {
        const int tn = min(TT, t_end - t0);
        // the previous tile's LDS reads are done (none before the first tile: its x loads then
        // issue right behind the row loads, without a fence waiting for those)
        if (t0 != t_begin) __syncthreads();
        // x tile into LDS, 4 loads per thread in flight before their LDS writes (clamped indices, no
        // branches, which would let the compiler sink each load to its write: past the end a thread
        // rewrites the last element with its own value)
        const int nx = tn * (n / 4);
        for (int i0 = threadIdx.x; i0 < nx; i0 += 4 * int(blockDim.x)) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = min(i0 + u * int(blockDim.x), nx - 1);
                const int t = i / (n / 4), k = (i % (n / 4)) * 4;
                v[u] = *reinterpret_cast<const float4*>(x + size_t(t0 + t) * n + k);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = min(i0 + u * int(blockDim.x), nx - 1);
                const int t = i / (n / 4), k = (i % (n / 4)) * 4;
                float* dst = xs + (t * 64 + k / L) * (L + 1) + k % L;   // L % 4 == 0: one chain
                dst[0] = v[u].x;
                dst[1] = v[u].y;
                dst[2] = v[u].z;
                dst[3] = v[u].w;
            }
        }
        __syncthreads();
        if (norm) {
            for (int t = wave; t < tn; t += int(blockDim.x >> 6)) {
                const float r = rms_scale_wave<L>(xs + (t * 64 + lane) * (L + 1), n);
                if (lane == 0) s_r[t] = r;
            }
            __syncthreads();
        }
        if (xq && blockIdx.y == 0) {   // Q8_0 of the layer input: item = (token, 32-block)
            const int hw = threadIdx.x >> 5, j = threadIdx.x & 31;
            const int nblk = tn * (n / kQ8);
            const int nhw = int(blockDim.x >> 5);
            for (int it = blockIdx.x * nhw + hw; it < nblk; it += gridDim.x * nhw) {
                const int t = it / (n / kQ8), k = (it % (n / kQ8)) * kQ8 + j;
                float v = xs[(t * 64 + k / L) * (L + 1) + k % L];
                if (norm) v = v * s_r[t];
                quant32(v, j, xq + size_t(t0 + t) * n + (k - j), xd + size_t(t0 + t) * (n / kQ8) + k / kQ8);
            }
        }
        if (!live) continue;
        for (int t = 0; t < tn; ++t) {
            const float* xc = xs + (t * 64 + lane) * (L + 1);
            float acc = 0.0f;
            if (norm) {
                const float r = s_r[t];
#pragma unroll
                for (int i = 0; i < L; ++i) {
                    const float u = xc[i] * r;
                    acc = fmaf(wr[i], u, acc);
                }
            } else {
#pragma unroll
                for (int i = 0; i < L; ++i) acc = fmaf(wr[i], xc[i], acc);
            }
            acc = wave_sum_tree(acc);
            if (lane == 0) {
                if (is_gate) gate[t0 + t] = acc;
                else logits[size_t(t0 + t) * E + row] = bias ? acc + b : acc;
            }
        }
    }
}

// ---- u = x * r per token (canonical RMS scale), one wave per token (prefill inputs)
template <int L>
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, int T, float* __restrict__ u) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= T) return;
    const int n = 64 * L;
    float xc[L];
#pragma unroll
    for (int i = 0; i < L; ++i) xc[i] = x[size_t(t) * n + lane * L + i];
    const float r = rms_scale_wave<L>(xc, n);
#pragma unroll
    for (int i = 0; i < L; ++i) u[size_t(t) * n + lane * L + i] = xc[i] * r;
}

// ---- Q8_0 of activations: one wave per 2 blocks of 32 (quant/q2_0/q2_0.cpp:93-108).
// xq int8 [rows][n] natural order, xd [rows][n/32]. With xhi (and xlo): the activations a = q * d as
// fp16 in the prefill GEMM's operand order (perm256_pos), [rows][n]: xhi = fp16(a) and
// xlo = fp16(a - xhi), an exact pair (a has at most 7 + 11 significant bits).
__global__ void k_quant_q8(const float* __restrict__ x, int n_blocks, int8_t* __restrict__ xq, float* __restrict__ xd,
                           _Float16* __restrict__ xhi, _Float16* __restrict__ xlo, int n) {
    const int gw = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;   // global wave
    const int lane = threadIdx.x & 63;
    const int blk = gw * 2 + (lane >> 5);
    if (gw * 2 >= n_blocks) return;   // whole waves only (the max below is across the wave's rows)
    const bool live = blk < n_blocks;
    const int j = lane & 31;
    const float v = live ? x[size_t(blk) * kQ8 + j] : 0.0f;
    const float am = half_max(fabsf(v));
    const float d = q8_scale(am);
    const float id = q8_inv(d);
    const int q = q8_code(v, id);
    if (!live) return;
    if (xq) xq[size_t(blk) * kQ8 + j] = int8_t(q);
    const float dr = f16_round(d);
    if (xd && j == 0) xd[blk] = dr;
    if (xhi) {
        const size_t e = size_t(blk) * kQ8 + j;   // element index in the row-major [rows][n]
        const size_t pos = (e & ~size_t(255)) + perm256_pos(int(e & 255));
        const float a = float(q) * dr;
        const _Float16 hi = _Float16(a);
        xhi[pos] = hi;
        if (xlo) xlo[pos] = _Float16(a - float(hi));
    }
}

// ---- Q8_0 of activations into the prefill GEMM's exact (hi, lo) fp16 pairs, perm256_pos order: one
// wave per 256-element stretch, 4 consecutive elements per lane (8 lanes per Q8_0 block of 32). The
// pairs go through LDS so that each lane then writes 4 consecutive positions (8 bytes) of each.
// Same values as k_quant_q8 with xhi / xlo.
// x [rows][n] -> the pairs [rows][np] (np >= n a multiple of 256; positions n .. np - 1 are zeros),
// Q8_0 blocks of blk = 32 or 64 values (moe_q2::run's block64).
__global__ void __launch_bounds__(256) k_quant_pairs(const float* __restrict__ x, int n, int np, int n_stretch, int blk,
                                                     _Float16* __restrict__ xhi, _Float16* __restrict__ xlo) {
    __shared__ _Float16 sp[4][2][256];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int st = blockIdx.x * 4 + wave;
    if (st >= n_stretch) return;   // whole waves; no workgroup barrier below
    const int spr = np / 256, row = st / spr, col = (st % spr) * 256 + lane * 4;   // n % 4 == 0
    const float4 v4 = col < n ? *reinterpret_cast<const float4*>(x + size_t(row) * n + col) : make_float4(0, 0, 0, 0);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = fmaxf(am, __shfl_xor(am, 1));
    am = fmaxf(am, __shfl_xor(am, 2));
    am = fmaxf(am, __shfl_xor(am, 4));   // the 8 lanes of a 32-block
    const float am16 = fmaxf(am, __shfl_xor(am, 8));
    am = blk == 64 ? am16 : am;          // the 16 lanes of a 64-block
    const float d = q8_scale(am);
    const float id = q8_inv(d);
    const float dr = f16_round(d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = float(q8_code(v[i], id)) * dr;
        const _Float16 hi = _Float16(a);
        const int p = perm256_pos(lane * 4 + i);
        sp[wave][0][p] = hi;
        sp[wave][1][p] = _Float16(a - float(hi));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's LDS writes are done (lgkmcnt(0))
    __builtin_amdgcn_wave_barrier();
    const uint2 h = *reinterpret_cast<const uint2*>(&sp[wave][0][lane * 4]);
    const uint2 l = *reinterpret_cast<const uint2*>(&sp[wave][1][lane * 4]);
    *reinterpret_cast<uint2*>(xhi + size_t(st) * 256 + lane * 4) = h;
    *reinterpret_cast<uint2*>(xlo + size_t(st) * 256 + lane * 4) = l;
}
// (a zero block quantizes to codes 0 with d = 0: the pad reads as exact zeros)

// wave per token
template <int V>
__global__ void __launch_bounds__(256) k_route_topk(const float* __restrict__ logits, int T, int E, int K,
                                                    int32_t* __restrict__ ids, float* __restrict__ wts, uint32_t* counts,
                                                    uint32_t* tail, int tail_from) {
    __shared__ float cand_v[4][64];
    __shared__ int cand_id[4][64];
    const int wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave, lane = threadIdx.x & 63;
    if (t >= T) return;
    const int id = topk_wave<V>(logits + size_t(t) * E, E, K, ids + size_t(t) * K, wts + size_t(t) * K, cand_v[wave],
                                cand_id[wave]);
    if (lane < K) {
        if (counts) atomicAdd(counts + id, 1u);
        if (tail && t >= tail_from) atomicAdd(tail + id, 1u);
    }
}

// ---- the routing records of a layer call from its logits (logit e of token t at
// lg[(t * E + e) * ls]): probs [T][K] = exp(l - max) / sum_e exp(l_e - max) with the sum in double
// (moe_ref.cu:146-164), tail_counts += 1 per selection of tokens t >= tail_from. One wave per token.
__global__ void __launch_bounds__(64) k_layer_trace(const float* __restrict__ lg, int ls, const int32_t* __restrict__ ids,
                                                    int T, int E, int K, uint32_t* __restrict__ tail_counts, int tail_from,
                                                    float* __restrict__ probs) {
    const int t = blockIdx.x, lane = threadIdx.x;
    if (t >= T) return;
    const float* l = lg + size_t(t) * E * ls;
    float mx = -INFINITY;
    for (int e = lane; e < E; e += 64) mx = fmaxf(mx, l[size_t(e) * ls]);
    mx = wave_max(mx);
    double s = 0.0;
    for (int e = lane; e < E; e += 64) s += double(expf(l[size_t(e) * ls] - mx));
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane < K) {
        const int id = ids[t * K + lane];
        if (probs) probs[t * K + lane] = float(double(expf(l[size_t(id) * ls] - mx)) / s);
        if (tail_counts && t >= tail_from) atomicAdd(tail_counts + id, 1u);
    }
}

}  // namespace

// ---------------------------------------------------------------- host entry points

static int router_tile_tokens(int L) { return int(98304 / (size_t(64) * (L + 1) * 4)); }
// Whether router_logits can quantize the input of T tokens in the same launch (one token tile).
bool router_fused_fits(int T, int n) {
    if (n % 64 || n < 512 || n > 64 * 64 || (n / 64) % 8) return false;
    int TT = router_tile_tokens(n / 64);
    if (TT > 16) TT = 16;
    return T <= TT;
}

int router_logits(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                  float* logits, float* gate, hipStream_t stream, int norm, int8_t* xq, float* xd) {
    if (T < 1 || E < 1 || E > kMaxE || n % 64 || n < 64 || n > 64 * 64) return set_error(kErrShape, "router: shape T=%d E=%d n=%d", T, E, n);
    if (!x || !W || !logits || (gate_w && !gate)) return set_error(kErrNull, "router: null pointer");
    const int L = n / 64;
    const int rows = E + (gate_w ? 1 : 0);
    if (xq && T > 16) return set_error(kErrShape, "router: fused quantization is for T <= 16");
    // token tile: the LDS tile stays within 96 KB, but always holds a decode window (4 tokens)
    int TT = router_tile_tokens(L);
    if (TT > 16) TT = 16;
    if (TT < 4) TT = 4;
    if (T < TT) TT = T;
    const size_t smem = size_t(TT) * 64 * (L + 1) * 4;
    // small T: one tile per workgroup row (and the fused quantization); else 64 tokens per workgroup
    // with the 4 router rows kept in registers across its tiles
    const int tok_per_wg = T <= TT ? T : 64;
    if (xq && T > TT) return set_error(kErrShape, "router: fused quantization needs T <= %d", TT);
    const int wg_rows = T <= TT ? 2 : 4;   // decode: 2 rows per workgroup; token tiles: 4
    dim3 grid((rows + wg_rows - 1) / wg_rows, (T + tok_per_wg - 1) / tok_per_wg);
#define FRT_ROUTER_L(LL)                                                                                         \
    case LL:                                                                                                     \
        if (smem > 65536)                                                                                        \
            FRT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_router<LL>),                            \
                                        hipFuncAttributeMaxDynamicSharedMemorySize, int(smem)));                 \
        launch_timed("router_quant", k_router<LL>, grid, dim3(64 * wg_rows), smem, stream, x, T, W, bias, gate_w, E, \
                     logits, gate, TT, tok_per_wg, norm, xq, xd);                                                    \
        break;
    switch (L) {
        FRT_ROUTER_L(8) FRT_ROUTER_L(16) FRT_ROUTER_L(24) FRT_ROUTER_L(32) FRT_ROUTER_L(40) FRT_ROUTER_L(48)
        FRT_ROUTER_L(56) FRT_ROUTER_L(64)
        default: return set_error(kErrShape, "router: n=%d needs n/64 in {8,16,..,64}", n);
    }
#undef FRT_ROUTER_L
    FRT_LAUNCHED("router_logits");
    return kOk;
}

int rmsnorm(const float* x, int T, int n, float* u, hipStream_t stream) {
    const unsigned grid = unsigned((T + 3) / 4);
    switch (n / 64) {
        case 8: k_rmsnorm<8><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 24: k_rmsnorm<24><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 56: k_rmsnorm<56><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 32: k_rmsnorm<32><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 40: k_rmsnorm<40><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 16: k_rmsnorm<16><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 48: k_rmsnorm<48><<<grid, 256, 0, stream>>>(x, T, u); break;
        case 64: k_rmsnorm<64><<<grid, 256, 0, stream>>>(x, T, u); break;
        default: return set_error(kErrShape, "rmsnorm: n=%d", n);
    }
    FRT_LAUNCHED("rmsnorm");
    return kOk;
}

// The prefill GEMM's activation pairs alone: rows of np (a multiple of 256, >= n) in perm256 order,
// Q8_0 blocks of blk (32 or 64) values.
int quantize_pairs(const float* x, int rows, int n, int np, int blk, _Float16* xhi, _Float16* xlo, hipStream_t stream) {
    if (rows < 1 || n % 128 || np % 256 || np < n || (blk != 32 && blk != 64))
        return set_error(kErrShape, "quantize_pairs: n=%d np=%d blk=%d", n, np, blk);
    const int ns = rows * (np / 256);
    launch_timed("pf_quant_x", k_quant_pairs, dim3((ns + 3) / 4), dim3(256), 0, stream, x, n, np, ns, blk, xhi, xlo);
    FRT_LAUNCHED("quantize_pairs");
    return kOk;
}

int quantize_q8(const float* x, int rows, int n, int8_t* xq, float* xd, _Float16* xhi, _Float16* xlo,
                hipStream_t stream) {
    if (rows < 1 || n % 64) return set_error(kErrShape, "quantize_q8: n=%d not a multiple of 64", n);
    const int nb = rows * (n / kQ8);
    if (xhi && xlo && !xq && !xd && n % 256 == 0) return quantize_pairs(x, rows, n, n, 32, xhi, xlo, stream);
    const int waves = (nb + 1) / 2;
    launch_timed("pf_quant_x", k_quant_q8, dim3((waves + 3) / 4), dim3(256), 0, stream, x, nb, xq, xd, xhi, xlo, n);
    FRT_LAUNCHED("quantize_q8");
    return kOk;
}

int route_topk(hipStream_t stream, const float* logits, int T, int E, int K, int32_t* ids, float* wts, uint32_t* counts,
               uint32_t* tail_counts, int tail_from) {
    if (E > kMaxE || E < 1 || K > 32 || K < 1 || K > E || T < 0 || (E <= 512 ? K > 64 : false)) return set_error(kErrShape, "moe_route_topk: unsupported shape E=%d k=%d", E, K);
    if (T == 0) return kOk;
    if (!logits || !ids || !wts) return set_error(kErrNull, "moe_route_topk: null pointer");
    const unsigned grid = unsigned((T + 3) / 4);
    if (E <= 512) k_route_topk<8><<<grid, 256, 0, stream>>>(logits, T, E, K, ids, wts, counts, tail_counts, tail_from);
    else k_route_topk<16><<<grid, 256, 0, stream>>>(logits, T, E, K, ids, wts, counts, tail_counts, tail_from);
    FRT_LAUNCHED("moe_route_topk");
    return kOk;
}

}  // namespace frt

// ---------------------------------------------------------------- prefill router GEMM
namespace frt {
namespace {

// logits [T][E] (and the shared gate [T] as row E) for many tokens in the canonical order, as a
// K-split GEMM that follows the order's own tree: the adjacent pairwise tree over the 64 chains is
// ((S0 + S1) + (S2 + S3)) + ((S4 + S5) + (S6 + S7)) with S_s the tree over chains 8 s .. 8 s + 7,
// so workgroup split s computes S_s and k_router_combine forms the top three levels (and adds the
// bias) exactly. (Eight splits rather than four: 2304 workgroups at T = 2048 fill whole rounds of
// the three per CU, and each thread keeps one level less of pending subtrees.)
// Within a split, K runs in natural order in tiles of L = n / 64 (one chain each); after each tile
// the chain sum joins a pairwise-tree stack (a binary counter: chain j merges with the completed
// subtrees named by the trailing one bits of j + 1).
// Workgroup tile 64 tokens x 64 rows, 256 threads, 4 x 4 outputs per thread; x and W tiles in LDS
// as [k][64 (+4 pad)] (a thread reads its 4 tokens and 4 rows as one float4 each); the next chain's tiles
// are loaded into registers while the current one is multiplied.
constexpr int kRgSplit = 8, kRgChains = 64 / kRgSplit, kRgLevels = 3;   // kRgChains = 2^kRgLevels

template <int L>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
k_router_gemm(const float* __restrict__ x, int T, const float* __restrict__ W, const float* __restrict__ gate_w, int E,
                                                     float* __restrict__ part) {
    // [k][64 + 4]: the transposing writes of 8 lanes (same row, 8 k) land in distinct bank groups
    __shared__ __align__(16) float sx[2][L][68];
    __shared__ __align__(16) float sw[2][L][68];
    const int n = 64 * L;
    const int E1 = E + (gate_w ? 1 : 0);
    const int t0 = blockIdx.y * 64, e0 = blockIdx.x * 64, c0 = blockIdx.z * kRgChains;
    const int tid = threadIdx.x;
    const int tr = (tid & 15) * 4, er = (tid >> 4) * 4;   // this thread's 4 tokens and 4 rows
    float lv[4][4][kRgLevels];   // pending subtrees of the levels below the split's root
    constexpr int F4 = L / 4;                    // float4 per row and chain
    constexpr int NP = (64 * F4 + 255) / 256;    // staging passes
    float4 rx[NP], rw[NP];
    auto load = [&](int c) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int idx = p * 256 + tid;
            const int row = idx / F4, q = idx % F4;
            const int t = min(t0 + row, T - 1), e = e0 + row;
            const float* wrow = e < E ? W + size_t(e) * n : gate_w;   // row E: the gate vector
            const bool in = idx < 64 * F4;
            rx[p] = in ? *reinterpret_cast<const float4*>(x + size_t(t) * n + c * L + q * 4) : make_float4(0, 0, 0, 0);
            rw[p] = in && e < E1 ? *reinterpret_cast<const float4*>(wrow + c * L + q * 4) : make_float4(0, 0, 0, 0);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int idx = p * 256 + tid;
            if (idx >= 64 * F4) continue;
            const int row = idx / F4, q = idx % F4;
            sx[buf][q * 4 + 0][row] = rx[p].x;
            sx[buf][q * 4 + 1][row] = rx[p].y;
            sx[buf][q * 4 + 2][row] = rx[p].z;
            sx[buf][q * 4 + 3][row] = rx[p].w;
            sw[buf][q * 4 + 0][row] = rw[p].x;
            sw[buf][q * 4 + 1][row] = rw[p].y;
            sw[buf][q * 4 + 2][row] = rw[p].z;
            sw[buf][q * 4 + 3][row] = rw[p].w;
        }
    };
    load(c0);
    store(0);
    __syncthreads();
    float total[4][4];
    for (int c = 0; c < kRgChains; ++c) {
        const int buf = c & 1;
        if (c + 1 < kRgChains) load(c0 + c + 1);
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
#pragma unroll 8
        for (int k = 0; k < L; ++k) {
            const float4 xv = *reinterpret_cast<const float4*>(&sx[buf][k][tr]);
            const float4 wv = *reinterpret_cast<const float4*>(&sw[buf][k][er]);
            const float xa[4] = {xv.x, xv.y, xv.z, xv.w}, wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(wa[j], xa[i], acc[i][j]);
        }
        // chain c joins the tree: for each level m while bit m of c is set, merge with the pending
        // left subtree of that level; the first clear bit parks the value there (uniform branches)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v = acc[i][j];
                bool parked = false;
#pragma unroll
                for (int m = 0; m < kRgLevels; ++m) {
                    if (parked) continue;
                    if (((c >> m) & 1) == 0) {
                        lv[i][j][m] = v;
                        parked = true;
                    } else {
                        v = lv[i][j][m] + v;
                    }
                }
                if (!parked) total[i][j] = v;   // the split's last chain: its whole subtree
            }
        if (c + 1 < kRgChains) {
            store(buf ^ 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + tr + i, e = e0 + er + j;
            if (t < T && e < E1) part[(size_t(blockIdx.z) * T + t) * E1 + e] = total[i][j];
        }
}

// top of the tree: v = ((S0 + S1) + (S2 + S3)) + ((S4 + S5) + (S6 + S7)); logits [T][E] = v + bias,
// gate [T] = row E's v
// The same split GEMM on the matrix cores. v_mfma_f32_16x16x4f32 accumulates its four products in
// K order as a chain of fused multiply-adds (d = fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0, c)))),
// bit for bit; checked on the MI355X over 5.12M random operands with exponents spread over 2^-12 ..
// 2^12), so a chain of L = n / 64 values is L / 4 MFMA steps from a zero accumulator in natural K
// order: the canonical chain exactly. The chains then join the same pending-subtree tree as above.
// Workgroup: 64 router rows x 64 tokens, 4 waves of 2 x 2 tiles of 16 x 16; per chain the W and x
// tiles are staged in LDS (row stride L + 4 floats: the 16 rows x 4 K of an operand read fall in
// distinct banks), the next chain's tiles loaded into registers during the current one's steps.
typedef float f32x4v __attribute__((ext_vector_type(4)));
template <int L>
__global__ void __launch_bounds__(256) k_router_mfma(const float* __restrict__ x, int T, const float* __restrict__ W,
                                                     const float* __restrict__ gate_w, int E, float* __restrict__ part) {
    // LDS row stride (floats): L + 2 = 2 mod 4 with (L + 2) / 2 odd, so the 16 rows x 2 K lanes of
    // each half-wave's operand read hit 32 distinct banks (rows 8 apart no longer share one)
    constexpr int LS = L + 2;
    constexpr int F4 = L / 4;                  // float4 per row and chain
    constexpr int NP = (64 * F4 + 255) / 256;  // staging passes
    __shared__ __align__(16) float sx[2][64 * LS];
    __shared__ __align__(16) float sw[2][64 * LS];
    const int E1 = E + (gate_w ? 1 : 0);
    const int t0 = blockIdx.y * 64, e0 = blockIdx.x * 64, c0 = blockIdx.z * kRgChains;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const int wr = (wave & 1) * 32, wc = (wave >> 1) * 32;   // this wave's rows and tokens in the tile
    const int n = 64 * L;
    float4 rx[NP], rw[NP];
    auto load = [&](int c) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int idx = p * 256 + tid;
            const int row = idx / F4, q = idx % F4;
            const int t = min(t0 + row, T - 1), e = e0 + row;
            const float* wrow = e < E ? W + size_t(e) * n : gate_w;   // row E: the gate vector
            const bool in = idx < 64 * F4;
            rx[p] = in ? *reinterpret_cast<const float4*>(x + size_t(t) * n + c * L + q * 4) : make_float4(0, 0, 0, 0);
            rw[p] = in && e < E1 ? *reinterpret_cast<const float4*>(wrow + c * L + q * 4) : make_float4(0, 0, 0, 0);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int idx = p * 256 + tid;
            if (idx >= 64 * F4) continue;
            const int row = idx / F4, q = idx % F4;
            float2* dx = reinterpret_cast<float2*>(&sx[buf][row * LS + q * 4]);   // (8-byte aligned rows)
            float2* dw = reinterpret_cast<float2*>(&sw[buf][row * LS + q * 4]);
            dx[0] = make_float2(rx[p].x, rx[p].y);
            dx[1] = make_float2(rx[p].z, rx[p].w);
            dw[0] = make_float2(rw[p].x, rw[p].y);
            dw[1] = make_float2(rw[p].z, rw[p].w);
        }
    };
    load(c0);
    store(0);
    __syncthreads();
    f32x4v lv[2][2][kRgLevels];   // pending subtrees of the levels below the split's root
    f32x4v total[2][2];
    for (int c = 0; c < kRgChains; ++c) {
        const int buf = c & 1;
        if (c + 1 < kRgChains) load(c0 + c + 1);
        f32x4v ch[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) ch[i][j] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
        const float* aw = &sw[buf][(wr + li) * LS + lg];
        const float* ax = &sx[buf][(wc + li) * LS + lg];
#pragma unroll
        for (int s = 0; s < L / 4; ++s) {
            const float a0 = aw[4 * s], a1 = aw[16 * LS + 4 * s];
            const float b0 = ax[4 * s], b1 = ax[16 * LS + 4 * s];
            ch[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, ch[0][0], 0, 0, 0);
            ch[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, ch[0][1], 0, 0, 0);
            ch[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, ch[1][0], 0, 0, 0);
            ch[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, ch[1][1], 0, 0, 0);
        }
        // chain c joins the tree (the same rule as k_router_gemm)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                f32x4v v = ch[i][j];
                bool parked = false;
#pragma unroll
                for (int m = 0; m < kRgLevels; ++m) {
                    if (parked) continue;
                    if (((c >> m) & 1) == 0) {
                        lv[i][j][m] = v;
                        parked = true;
                    } else {
                        v = lv[i][j][m] + v;
                    }
                }
                if (!parked) total[i][j] = v;
            }
        if (c + 1 < kRgChains) {
            store(buf ^ 1);
            __syncthreads();
        }
    }
    // lane: router rows 4 lg + v of row tile i, token li of token tile j
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t = t0 + wc + 16 * j + li;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int e = e0 + wr + 16 * i + 4 * lg + v;
                if (t < T && e < E1) part[(size_t(blockIdx.z) * T + t) * E1 + e] = total[i][j][v];
            }
        }
}

__global__ void __launch_bounds__(256) k_router_combine(const float* __restrict__ part, int T, int E, int E1,
                                                        const float* __restrict__ bias, float* __restrict__ logits,
                                                        float* __restrict__ gate) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x, N = size_t(T) * E1;
    if (i >= N) return;
    const int t = int(i / E1), e = int(i % E1);
    const float v = ((part[i] + part[N + i]) + (part[2 * N + i] + part[3 * N + i])) +
                    ((part[4 * N + i] + part[5 * N + i]) + (part[6 * N + i] + part[7 * N + i]));
    if (e < E) logits[size_t(t) * E + e] = bias ? v + bias[e] : v;
    else gate[t] = v;
}

// k_router_combine and k_route_topk in one pass (E <= 512): wave w of a workgroup takes token
// 4 blockIdx.x + w, sums its logits from the split's partials in k_router_combine's tree (writing the
// logits and the gate as it does) into LDS, and selects from there with the same topk_wave.
__global__ void __launch_bounds__(256) k_route_topk_part(const float* __restrict__ part, int T, int E, int E1,
                                                         const float* __restrict__ bias, float* __restrict__ logits,
                                                         float* __restrict__ gate, int K, int32_t* __restrict__ ids,
                                                         float* __restrict__ wts, uint32_t* counts) {
    __shared__ __align__(16) float row[4][512];
    __shared__ float cand_v[4][64];
    __shared__ int cand_id[4][64];
    const int wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave, lane = threadIdx.x & 63;
    if (t >= T) return;   // (whole waves; no workgroup barrier below)
    const size_t N = size_t(T) * E1;
    for (int e = lane; e < E1; e += 64) {
        const size_t i = size_t(t) * E1 + e;
        const float v = ((part[i] + part[N + i]) + (part[2 * N + i] + part[3 * N + i])) +
                        ((part[4 * N + i] + part[5 * N + i]) + (part[6 * N + i] + part[7 * N + i]));
        if (e < E) {
            const float l = bias ? v + bias[e] : v;
            logits[size_t(t) * E + e] = l;
            row[wave][e] = l;
        } else {
            gate[t] = v;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int id = topk_wave<8>(row[wave], E, K, ids + size_t(t) * K, wts + size_t(t) * K, cand_v[wave], cand_id[wave]);
    if (lane < K && counts) atomicAdd(counts + id, 1u);
}

}  // namespace

int g_router_mfma = 1;   // the prefill router GEMM on the matrix cores (0: the VALU kernel)

size_t router_gemm_ws_bytes(int T, int E, bool gate) { return size_t(kRgSplit) * T * (E + (gate ? 1 : 0)) * 4; }

// the K-split partial sums of the router GEMM (logits and gate before the combine)
static int router_gemm_part(const float* x, int T, const float* W, const float* gate_w, int E, int n, float* gate,
                            float* part, hipStream_t stream) {
    if (n % 512 || n < 512 || n > 4096) return set_error(kErrShape, "router_gemm: n=%d (a multiple of 512 up to 4096)", n);
    if (T < 1 || E < 1 || !part || (gate_w && !gate)) return set_error(kErrShape, "router_gemm: T=%d E=%d", T, E);
    const int E1 = E + (gate_w ? 1 : 0);
    dim3 grid((E1 + 63) / 64, (T + 63) / 64, kRgSplit);
    if (g_router_mfma) {
        switch (n / 64) {
            case 8: launch_timed("router_gemm", k_router_mfma<8>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 16: launch_timed("router_gemm", k_router_mfma<16>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 24: launch_timed("router_gemm", k_router_mfma<24>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 56: launch_timed("router_gemm", k_router_mfma<56>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 32: launch_timed("router_gemm", k_router_mfma<32>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 40: launch_timed("router_gemm", k_router_mfma<40>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 48: launch_timed("router_gemm", k_router_mfma<48>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 64: launch_timed("router_gemm", k_router_mfma<64>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            default: return set_error(kErrShape, "router_gemm: n=%d", n);
        }
    } else {
        switch (n / 64) {
            case 8: launch_timed("router_gemm", k_router_gemm<8>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 16: launch_timed("router_gemm", k_router_gemm<16>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 24: launch_timed("router_gemm", k_router_gemm<24>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 56: launch_timed("router_gemm", k_router_gemm<56>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 32: launch_timed("router_gemm", k_router_gemm<32>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 40: launch_timed("router_gemm", k_router_gemm<40>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 48: launch_timed("router_gemm", k_router_gemm<48>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            case 64: launch_timed("router_gemm", k_router_gemm<64>, grid, dim3(256), 0, stream, x, T, W, gate_w, E, part); break;
            default: return set_error(kErrShape, "router_gemm: n=%d", n);
        }
    }
    FRT_LAUNCHED("router_gemm");
    return kOk;
}

int router_gemm(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                float* logits, float* gate, float* part, hipStream_t stream) {
    if (int rc = router_gemm_part(x, T, W, gate_w, E, n, gate, part, stream)) return rc;
    const int E1 = E + (gate_w ? 1 : 0);
    const size_t N = size_t(T) * E1;
    k_router_combine<<<unsigned((N + 255) / 256), 256, 0, stream>>>(part, T, E, E1, bias, logits, gate);
    FRT_LAUNCHED("router_combine");
    return kOk;
}

// router_gemm then route_topk, the partials' combine fused into the selection where E <= 512
int router_gemm_topk(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                     float* logits, float* gate, float* part, int K, int32_t* ids, float* wts, uint32_t* counts,
                     hipStream_t stream) {
    if (E > 512 || K > 32 || K < 1 || K > E || !ids || !wts) {   // (route_topk's own checks and errors)
        if (int rc = router_gemm(x, T, W, bias, gate_w, E, n, logits, gate, part, stream)) return rc;
        return route_topk(stream, logits, T, E, K, ids, wts, counts, nullptr, 1 << 30);
    }
    if (int rc = router_gemm_part(x, T, W, gate_w, E, n, gate, part, stream)) return rc;
    const int E1 = E + (gate_w ? 1 : 0);
    launch_timed("route_topk", k_route_topk_part, dim3((T + 3) / 4), dim3(256), 0, stream, (const float*)part, T, E, E1,
                 bias, logits, gate, K, ids, wts, counts);
    FRT_LAUNCHED("router combine + top-k");
    return kOk;
}

int layer_trace(const float* lg, int ls, const int32_t* ids, int T, int E, int K, uint32_t* tail_counts, int tail_from,
                float* probs, hipStream_t stream) {
    if (T < 1) return kOk;
    k_layer_trace<<<T, 64, 0, stream>>>(lg, ls, ids, T, E, K, tail_counts, tail_from, probs);
    FRT_LAUNCHED("layer trace");
    return kOk;
}

}  // namespace frt
