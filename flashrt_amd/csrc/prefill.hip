// Prefill MoE: routed (token, slot) pairs sorted by expert, then grouped GEMMs on fp16 MFMA
// (kernels/cuda/moe_q2.cu:514-548 is the reference's int8 counterpart).
//
// Dispatch (moe_q2.cu:83-168 semantics: a stable sort of slots s = t*K + k by ids[s]):
//   k_pf_hist   per chunk of 1024 slots, an LDS histogram of experts (integer atomics only)
//   k_pf_scan   one workgroup: per-expert column prefix over chunks, bounds, the tile list
//   k_pf_place  one wave per chunk walks its slots in order, 64 at a time; each lane's rank among
//               equal experts in the batch comes from ballots (a wave64 match-any), so the
//               placement is stable and needs no atomics.
//   The shared expert, when present, is group E holding every token in order (rows T*K + t).
//
// GEMMs. Operands are exact in fp16: weights (q - 1) * d_w (a small integer times an fp16 scale)
// and activation codes (int8). One v_mfma_f32_16x16x32_f16 covers exactly one 32-value
// activation block, so its result (exact: integer multiples of d_w's ulp below 2^24) is scaled by
// that block's d_a with one fp32 FMA: the float error is that of an fp32 dot product, and the Q8_0
// quantization of h matches the CPU path's almost everywhere.
//   K order of a 64-block as the MFMA lanes use it (perm64): half h, lane group g, slot i ->
//   element 16 s + 4 g + c with s = 2h + i/4, c = (0, 2, 1, 3)[i % 4]; lane group g of a weight
//   row then needs only code dword g of the block. Activations are stored in this order.
//   k_pf_gateup  tile (64 tokens of one group) x 64 ff rows: gate and up, SwiGLU, Q8_0 of h
//   k_pf_down    tile x 64 output rows: down -> yd[slot][n]
//   k_pf_combine out[t] = sum_k (in expert order) w * yd[t*K+k] + yd[shared t] * sigmoid(gate)
#include "common.hpp"

#include <hip/hip_bf16.h>

namespace frt {

constexpr int kTN = 64;        // tokens per GEMM tile
constexpr int kChunk = 1024;   // slots per dispatch chunk

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

// ---------------------------------------------------------------- dispatch

__global__ void __launch_bounds__(256) k_pf_hist(const int32_t* __restrict__ ids, int S, int E, int32_t* __restrict__ cnt) {
    extern __shared__ int32_t h[];
    for (int e = threadIdx.x; e < E; e += blockDim.x) h[e] = 0;
    __syncthreads();
    const int s0 = blockIdx.x * kChunk, s1 = min(S, s0 + kChunk);
    for (int s = s0 + threadIdx.x; s < s1; s += blockDim.x) {
        const int e = ids[s];
        if (unsigned(e) < unsigned(E)) atomicAdd(&h[e], 1);   // ids outside [0, E) are dropped
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[size_t(blockIdx.x) * E + e] = h[e];
}

__device__ __forceinline__ int block_excl_scan(int v, int* total, int* ws) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) ws[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int w = 0; w < nw; ++w) {
            const int x = ws[w];
            ws[w] = run;
            run += x;
        }
        ws[nw] = run;
    }
    __syncthreads();
    const int r = ws[wave] + incl - v;
    *total = ws[nw];
    __syncthreads();
    return r;
}

// 1024 threads. cnt [nchunk][E] becomes each chunk's first row per expert (absolute).
__global__ void __launch_bounds__(1024) k_pf_scan(int32_t* __restrict__ cnt, int nchunk, int E, int T, int K, int shared,
                                                  int32_t* __restrict__ bounds, int2* __restrict__ tiles,
                                                  int32_t* __restrict__ n_tiles) {
    __shared__ int ws[17];
    int run_rows = 0, run_tiles = 0;
    for (int e0 = 0; e0 < E; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        int c = 0;
        if (e < E)
            for (int b = 0; b < nchunk; ++b) c += cnt[size_t(b) * E + e];
        int tot_rows, tot_tiles;
        const int off = block_excl_scan(c, &tot_rows, ws) + run_rows;
        const int nt = (c + kTN - 1) / kTN;
        const int toff = block_excl_scan(nt, &tot_tiles, ws) + run_tiles;
        if (e < E) {
            bounds[e] = off;
            for (int i = 0; i < nt; ++i) tiles[toff + i] = make_int2(e, i * kTN);
            int run = off;
            for (int b = 0; b < nchunk; ++b) {
                const int x = cnt[size_t(b) * E + e];
                cnt[size_t(b) * E + e] = run;
                run += x;
            }
        }
        run_rows += tot_rows;
        run_tiles += tot_tiles;
    }
    if (threadIdx.x == 0) {
        bounds[E] = run_rows;   // = T * K
        int nt = run_tiles;
        if (shared) {
            bounds[E + 1] = run_rows + T;
            for (int j = 0; j < T; j += kTN) tiles[nt++] = make_int2(E, j);
        }
        *n_tiles = nt;
    }
}

// one wave per chunk; stable ranks from a ballot match-any over the expert id bits
__global__ void __launch_bounds__(64) k_pf_place(const int32_t* __restrict__ ids, int S, int K, int E, int id_bits,
                                                 const int32_t* __restrict__ cnt, int32_t* __restrict__ tok_of,
                                                 int32_t* __restrict__ slot_of) {
    extern __shared__ int32_t next[];
    const int lane = threadIdx.x;
    for (int e = lane; e < E; e += 64) next[e] = cnt[size_t(blockIdx.x) * E + e];
    __syncthreads();
    const int s0 = blockIdx.x * kChunk, s1 = min(S, s0 + kChunk);
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int b = s0; b < s1; b += 64) {
        const int s = b + lane;
        const int e0 = s < s1 ? ids[s] : -1;
        const bool valid = unsigned(e0) < unsigned(E);
        const int e = valid ? e0 : 0;
        uint64_t peers = __ballot(valid);
        for (int bit = 0; bit < id_bits; ++bit) {
            const bool on = (e >> bit) & 1;
            const uint64_t m = __ballot(on);
            peers &= on ? m : ~m;
        }
        if (valid) {
            const int rank = __popcll(peers & lt);
            const int row = next[e] + rank;
            tok_of[row] = s / K;
            slot_of[row] = s;
            if (rank == 0) next[e] += __popcll(peers);   // the first lane of each expert
        }
        __syncthreads();
    }
}

__global__ void k_pf_place_shared(int T, int K, int32_t* __restrict__ tok_of, int32_t* __restrict__ slot_of) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < T) {
        tok_of[T * K + t] = t;
        slot_of[T * K + t] = T * K + t;
    }
}

// ---------------------------------------------------------------- GEMM pieces

// A operand (8 fp16) of half h for one weight row's code dword g (see perm64 above), scaled by d.
__device__ __forceinline__ half8 dequant8(uint32_t cw, int h, _Float16 d) {
    const half2v one025 = {_Float16(1025.0f), _Float16(1025.0f)};
    const half2v dd = {d, d};
    half8 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int sh = 4 * h + ((k & 2) ? 2 : 0) + ((k & 1) ? 8 : 0);
        const uint32_t x = ((cw >> sh) & 0x00030003u) | 0x64006400u;   // fp16 1024 + q in both halves
        half2v v = __builtin_bit_cast(half2v, x);
        v = (v - one025) * dd;                                        // (q - 1) * d, exact
        r[2 * k] = v[0];
        r[2 * k + 1] = v[1];
    }
    return r;
}

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b) {
    const floatx4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, z, 0, 0, 0);
}

// position of element e (0..63) of a 64-block in the perm64 order
__device__ __forceinline__ int perm64_pos(int e) {
    const int s = e >> 4, g = (e >> 2) & 3, c = e & 3;
    const int ci = c == 0 ? 0 : c == 1 ? 2 : c == 2 ? 1 : 3;
    return (s >> 1) * 32 + g * 8 + (s & 1) * 4 + ci;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// ---------------------------------------------------------------- gate + up

constexpr int kKC = 128;   // K per LDS stage (2 blocks)

// grid (ff / 64, max_tiles); 256 threads: wave w owns ff rows f0 + 16w .. +15 (gate and up).
__global__ void __launch_bounds__(256) k_pf_gateup(const uint8_t* __restrict__ arena, size_t stride, int E,
                                                   const uint8_t* __restrict__ shared_blob, int n, int ff,
                                                   const _Float16* __restrict__ xq16, const float* __restrict__ xd,
                                                   const int32_t* __restrict__ tok_of, const int32_t* __restrict__ bounds,
                                                   const int2* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                   _Float16* __restrict__ hq16, float* __restrict__ hd) {
    if (int(blockIdx.y) >= *n_tiles) return;
    const int2 tile = tiles[blockIdx.y];
    const int grp = tile.x;
    const int row0 = bounds[grp] + tile.y;
    const int cnt = min(kTN, bounds[grp + 1] - row0);
    const uint8_t* blob = grp < E ? arena + size_t(grp) * stride : shared_blob;
    const int nb = n / kBlock;
    const int f0 = blockIdx.x * 64;
    const size_t mb = mat_bytes(ff, n);

    __shared__ __align__(16) uint32_t sA[128][kKC / 64][4];   // codes: row, block, dword
    __shared__ uint16_t sS[128][kKC / 64];                    // weight scales
    __shared__ __align__(16) _Float16 sB[kTN][kKC + 8];       // activation codes (perm64 order)
    __shared__ float sD[kTN][kKC / 32];                       // activation scales
    __shared__ int sTok[kTN];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid < kTN) sTok[tid] = tid < cnt ? tok_of[row0 + tid] : -1;
    __syncthreads();

    floatx4 acc[2][4];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[m][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    const int li = lane & 15, lg = lane >> 4;
    for (int k0 = 0; k0 < n; k0 += kKC) {
        const int b0 = k0 / kBlock;
        // stage A: 128 rows x 2 blocks x 16 B (one uint4 per thread), scales
        {
            const int r = tid >> 1, bb = tid & 1;
            const uint8_t* base = blob + (r < 64 ? 0 : mb);
            const int fr = f0 + (r & 63);
            const uint4 v = *reinterpret_cast<const uint4*>(base + (size_t(fr) * nb + b0 + bb) * 16);
            *reinterpret_cast<uint4*>(&sA[r][bb][0]) = v;
            const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + size_t(ff) * nb * 16);
            sS[r][bb] = sc[size_t(fr) * nb + b0 + bb];
        }
        // stage B: 64 tokens x 128 fp16 (16 uint4 per token), scales 64 x 4
        for (int i = tid; i < kTN * (kKC / 8); i += 256) {
            const int j = i / (kKC / 8), q = i % (kKC / 8);
            const int t = sTok[j];
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t >= 0) v = *reinterpret_cast<const uint4*>(xq16 + size_t(t) * n + k0 + q * 8);
            *reinterpret_cast<uint4*>(&sB[j][q * 8]) = v;
        }
        {
            const int j = tid >> 2, q = tid & 3;
            const int t = sTok[j];
            sD[j][q] = t >= 0 ? xd[size_t(t) * (n / kQ8) + k0 / kQ8 + q] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int bb = 0; bb < kKC / 64; ++bb) {
            const int ra = wave * 16 + li;   // gate row in the tile; up row = ra + 64
            const uint32_t cg = sA[ra][bb][lg], cu = sA[64 + ra][bb][lg];
            const _Float16 dg = __builtin_bit_cast(_Float16, sS[ra][bb]);
            const _Float16 du = __builtin_bit_cast(_Float16, sS[64 + ra][bb]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const half8 ag = dequant8(cg, h, dg), au = dequant8(cu, h, du);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int col = t * 16 + li;
                    const half8 b = *reinterpret_cast<const half8*>(&sB[col][bb * 64 + h * 32 + lg * 8]);
                    const float da = sD[col][bb * 2 + h];
                    const floatx4 cgv = mfma16(ag, b), cuv = mfma16(au, b);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[0][t][j] = fmaf(cgv[j], da, acc[0][t][j]);
                        acc[1][t][j] = fmaf(cuv[j], da, acc[1][t][j]);
                    }
                }
            }
        }
        __syncthreads();
    }
    // SwiGLU into LDS: hbuf[token][ff row in tile]; D layout: lane -> col li, rows 4*lg + j
    float* hbuf = reinterpret_cast<float*>(&sB[0][0]);   // 64 x 64 floats = 16 KB (sB is 17 KB)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) hbuf[(t * 16 + li) * 64 + wave * 16 + lg * 4 + j] = silu_mul(acc[0][t][j], acc[1][t][j]);
    __syncthreads();
    // Q8_0 per (token, 32-row block): half-wave per pair
    const int hw = tid >> 5, hl = tid & 31;
    for (int p = hw; p < kTN * 2; p += 8) {
        const int j = p >> 1, qb = p & 1;
        if (j >= cnt) continue;
        const float v = hbuf[j * 64 + qb * 32 + hl];
        const float am = half_max(fabsf(v));
        const float d = q8_scale(am);
        const float id = q8_inv(d);
        const size_t row = size_t(row0 + j);
        hq16[row * ff + f0 + perm64_pos(qb * 32 + hl)] = _Float16(float(q8_code(v, id)));
        if (hl == 0) hd[row * (ff / kQ8) + f0 / kQ8 + qb] = f16_round(d);
    }
}

// ---------------------------------------------------------------- down

// grid (n / 64, max_tiles); 256 threads; the tile's h (64 tokens x ff, fp16) stays in LDS.
template <typename OutT>
__global__ void __launch_bounds__(256) k_pf_down(const uint8_t* __restrict__ arena, size_t stride, int E,
                                                 const uint8_t* __restrict__ shared_blob, int n, int ff,
                                                 const _Float16* __restrict__ hq16, const float* __restrict__ hd,
                                                 const int32_t* __restrict__ slot_of, const int32_t* __restrict__ bounds,
                                                 const int2* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                 OutT* __restrict__ yd) {
    if (int(blockIdx.y) >= *n_tiles) return;
    extern __shared__ __align__(16) uint8_t smem[];
    const int2 tile = tiles[blockIdx.y];
    const int grp = tile.x;
    const int row0 = bounds[grp] + tile.y;
    const int cnt = min(kTN, bounds[grp + 1] - row0);
    const uint8_t* blob = (grp < E ? arena + size_t(grp) * stride : shared_blob) + 2 * mat_bytes(ff, n);
    const int nbf = ff / kBlock;
    const int ldb = ff + 8;   // padded fp16 row
    _Float16* sB = reinterpret_cast<_Float16*>(smem);                             // [64][ldb]
    float* sD = reinterpret_cast<float*>(smem + size_t(kTN) * ldb * 2);           // [64][ff/32]
    uint32_t* sA = reinterpret_cast<uint32_t*>(sD + kTN * (ff / kQ8));            // [64 rows][nbf][4]
    uint16_t* sS = reinterpret_cast<uint16_t*>(sA + 64 * nbf * 4);                // [64][nbf]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = blockIdx.x * 64;
    for (int i = tid; i < kTN * (ff / 8); i += 256) {
        const int j = i / (ff / 8), q = i % (ff / 8);
        uint4 v = make_uint4(0, 0, 0, 0);
        if (j < cnt) v = *reinterpret_cast<const uint4*>(hq16 + size_t(row0 + j) * ff + q * 8);
        *reinterpret_cast<uint4*>(sB + j * ldb + q * 8) = v;
    }
    for (int i = tid; i < kTN * (ff / kQ8); i += 256) {
        const int j = i / (ff / kQ8);
        sD[i] = j < cnt ? hd[size_t(row0 + j) * (ff / kQ8) + i % (ff / kQ8)] : 0.0f;
    }
    for (int i = tid; i < 64 * nbf; i += 256) {
        const int r = i / nbf, b = i % nbf;
        *reinterpret_cast<uint4*>(sA + (r * nbf + b) * 4) =
            *reinterpret_cast<const uint4*>(blob + (size_t(r0 + r) * nbf + b) * 16);
        sS[i] = reinterpret_cast<const uint16_t*>(blob + size_t(n) * nbf * 16)[size_t(r0 + r) * nbf + b];
    }
    __syncthreads();
    const int li = lane & 15, lg = lane >> 4;
    const int ra = wave * 16 + li;
    floatx4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nbf; ++b) {
        const uint32_t cw = sA[(ra * nbf + b) * 4 + lg];
        const _Float16 d = __builtin_bit_cast(_Float16, sS[ra * nbf + b]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const half8 a = dequant8(cw, h, d);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int col = t * 16 + li;
                const half8 bv = *reinterpret_cast<const half8*>(sB + col * ldb + b * 64 + h * 32 + lg * 8);
                const float da = sD[col * (ff / kQ8) + 2 * b + h];
                const floatx4 c = mfma16(a, bv);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][j] = fmaf(c[j], da, acc[t][j]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int col = t * 16 + li;
        if (col >= cnt) continue;
        const size_t slot = size_t(slot_of[row0 + col]);
        OutT* dst = yd + slot * n + r0 + wave * 16 + lg * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[j] = OutT(acc[t][j]);
    }
}

// ---------------------------------------------------------------- combine

// out[t][i] = sum over the token's K slots in ascending expert id of w * yd (+ shared * sigmoid(g))
template <typename InT>
__global__ void __launch_bounds__(256) k_pf_combine(const InT* __restrict__ yd, const int32_t* __restrict__ ids,
                                                    const float* __restrict__ wts, const float* __restrict__ gate, int T,
                                                    int K, int n, int shared, const float* __restrict__ resid,
                                                    float* __restrict__ out) {
    __shared__ int order[32];
    const int t = blockIdx.y;
    if (threadIdx.x == 0) {
        int prev = -1;
        for (int r = 0; r < K; ++r) {   // selection order by expert id (ids of one token are distinct)
            int best = -1, bid = 0x7fffffff;
            for (int k = 0; k < K; ++k) {
                const int e = ids[t * K + k];
                if (e > prev && e < bid) {
                    bid = e;
                    best = k;
                }
            }
            order[r] = best;
            prev = bid;
        }
    }
    __syncthreads();
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float acc = 0.0f;
    for (int r = 0; r < K; ++r) {
        const int k = order[r];
        const float p = wts[t * K + k] * float(yd[(size_t(t) * K + k) * n + i]);
        acc = acc + p;
    }
    float o = acc;
    if (shared) {
        const float g = 1.0f / (1.0f + expf(-gate[t]));
        const float p = float(yd[(size_t(T) * K + t) * n + i]) * g;
        o = acc + p;
    }
    if (resid) o = resid[size_t(t) * n + i] + o;
    out[size_t(t) * n + i] = o;
}

}  // namespace

// ---------------------------------------------------------------- host side

struct PfWs {
    int32_t *cnt, *bounds, *tok_of, *slot_of, *n_tiles;
    int2* tiles;
    int8_t* xq;
    float* xd;
    _Float16* xq16;
    _Float16* hq16;
    float* hd;
    float* yd;   // only when the layer path owns it
    size_t bytes;
};

static int pf_max_tiles(int S, int G) { return (S + kTN - 1) / kTN + G; }

static PfWs pf_carve(void* base, int T, int K, int n, int ff, int E, bool shared, bool own_yd) {
    PfWs w{};
    uint8_t* p = static_cast<uint8_t*>(base);
    auto take = [&](size_t b) {
        uint8_t* r = p;
        p += up256(b);
        return r;
    };
    const int S = T * K + (shared ? T : 0);
    const int G = E + (shared ? 1 : 0);
    const int nchunk = (T * K + kChunk - 1) / kChunk;
    w.cnt = reinterpret_cast<int32_t*>(take(size_t(nchunk) * E * 4));
    w.bounds = reinterpret_cast<int32_t*>(take(size_t(E + 2) * 4));
    w.tok_of = reinterpret_cast<int32_t*>(take(size_t(S) * 4));
    w.slot_of = reinterpret_cast<int32_t*>(take(size_t(S) * 4));
    w.n_tiles = reinterpret_cast<int32_t*>(take(4));
    w.tiles = reinterpret_cast<int2*>(take(size_t(pf_max_tiles(S, G)) * 8));
    w.xq = reinterpret_cast<int8_t*>(take(size_t(T) * n));
    w.xd = reinterpret_cast<float*>(take(size_t(T) * (n / kQ8) * 4));
    w.xq16 = reinterpret_cast<_Float16*>(take(size_t(T) * n * 2));
    w.hq16 = reinterpret_cast<_Float16*>(take(size_t(S) * ff * 2));
    w.hd = reinterpret_cast<float*>(take(size_t(S) * (ff / kQ8) * 4));
    w.yd = own_yd ? reinterpret_cast<float*>(take(size_t(S) * n * 4)) : nullptr;
    w.bytes = size_t(p - static_cast<uint8_t*>(base));
    return w;
}

size_t pf_workspace_bytes(int T, int K, int n, int ff, int E, bool shared, bool own_yd) {
    return pf_carve(nullptr, T, K, n, ff, E, shared, own_yd).bytes + 256;
}

int quantize_q8(const float* x, int rows, int n, int8_t* xq, float* xd, _Float16* xq16, hipStream_t stream);

int pf_check(int T, int K, int n, int ff, int E) {
    if (T < 1 || K < 1 || K > 32 || E < 1 || E > 4096 || K > E) return set_error(kErrShape, "prefill: T=%d K=%d E=%d", T, K, E);
    if (n % 128 || ff % 64 || n < 128 || ff < 64 || ff > 4096) return set_error(kErrShape, "prefill: n=%d ff=%d (n %% 128, ff %% 64)", n, ff);
    return kOk;
}

// The grouped expert products for routed ids (+ optionally the shared expert as group E).
// yd_kind: 0 float, 1 bf16 (moe_q2::run's yd_bf16)
static int pf_experts(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff,
                      const float* x, const int32_t* ids, int T, int K, void* yd, int yd_kind, const PfWs& w,
                      hipStream_t stream) {
    const bool shared = shared_blob != nullptr;
    const int S = T * K + (shared ? T : 0);
    const int G = E + (shared ? 1 : 0);
    const int nchunk = (T * K + kChunk - 1) / kChunk;
    int id_bits = 1;
    while ((1 << id_bits) < E) ++id_bits;
    if (int rc = quantize_q8(x, T, n, w.xq, w.xd, w.xq16, stream)) return rc;
    timing_mark(stream, "pf_quant_x");
    k_pf_hist<<<nchunk, 256, size_t(E) * 4, stream>>>(ids, T * K, E, w.cnt);
    k_pf_scan<<<1, 1024, 0, stream>>>(w.cnt, nchunk, E, T, K, shared ? 1 : 0, w.bounds, w.tiles, w.n_tiles);
    k_pf_place<<<nchunk, 64, size_t(E) * 4, stream>>>(ids, T * K, K, E, id_bits, w.cnt, w.tok_of, w.slot_of);
    if (shared) k_pf_place_shared<<<(T + 255) / 256, 256, 0, stream>>>(T, K, w.tok_of, w.slot_of);
    timing_mark(stream, "pf_dispatch");
    const int mt = pf_max_tiles(S, G);
    k_pf_gateup<<<dim3(ff / 64, mt), 256, 0, stream>>>(arena, stride, E, shared_blob, n, ff, w.xq16, w.xd, w.tok_of,
                                                       w.bounds, w.tiles, w.n_tiles, w.hq16, w.hd);
    timing_mark(stream, "pf_gateup");
    const int nbf = ff / kBlock;
    const size_t smem = size_t(kTN) * (ff + 8) * 2 + size_t(kTN) * (ff / kQ8) * 4 + size_t(64) * nbf * 16 + size_t(64) * nbf * 2;
    if (yd_kind == 1) {
        FRT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_down<__hip_bfloat16>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(smem)));
        k_pf_down<__hip_bfloat16><<<dim3(n / 64, mt), 256, smem, stream>>>(arena, stride, E, shared_blob, n, ff, w.hq16, w.hd,
                                                                           w.slot_of, w.bounds, w.tiles, w.n_tiles,
                                                                           static_cast<__hip_bfloat16*>(yd));
    } else {
        FRT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_down<float>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(smem)));
        k_pf_down<float><<<dim3(n / 64, mt), 256, smem, stream>>>(arena, stride, E, shared_blob, n, ff, w.hq16, w.hd,
                                                                  w.slot_of, w.bounds, w.tiles, w.n_tiles,
                                                                  static_cast<float*>(yd));
    }
    timing_mark(stream, "pf_down");
    FRT_LAUNCHED("prefill experts");
    return kOk;
}

// moe_q2::run (kernels/cuda/moe_q2.h:20-30): yd [T*K][n] per slot
int pf_run(const uint8_t* experts, size_t stride, int E, int n, int ff, const float* x, const int32_t* ids, int T, int K,
           void* yd, void* ws, size_t ws_bytes, hipStream_t stream, int block64, int yd_bf16) {
    if (int rc = pf_check(T, K, n, ff, E)) return rc;
    if (block64) return set_error(kErrShape, "moe_q2::run: block64 activations are not supported (Q8_0 blocks of 32 only)");
    if (!experts || !x || !ids || !yd || !ws) return set_error(kErrNull, "moe_q2::run: null pointer");
    const PfWs w = pf_carve(ws, T, K, n, ff, E, false, false);
    if (w.bytes > ws_bytes) return set_error(kErrWorkspace, "moe_q2::run: workspace %zu < %zu", ws_bytes, w.bytes);
    return pf_experts(experts, stride, E, nullptr, n, ff, x, ids, T, K, yd, yd_bf16 ? 1 : 0, w, stream);
}

// The whole prefill layer after routing: ids/wts [T][K], gate [T] -> out [T][n] (+ resid)
int pf_moe(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff, const float* x,
           const int32_t* ids, const float* wts, const float* gate, int T, int K, const float* resid, float* out,
           void* ws, size_t ws_bytes, hipStream_t stream) {
    if (int rc = pf_check(T, K, n, ff, E)) return rc;
    const PfWs w = pf_carve(ws, T, K, n, ff, E, true, true);
    if (w.bytes > ws_bytes) return set_error(kErrWorkspace, "prefill: workspace %zu < %zu", ws_bytes, w.bytes);
    if (int rc = pf_experts(arena, stride, E, shared_blob, n, ff, x, ids, T, K, w.yd, 0, w, stream)) return rc;
    k_pf_combine<float><<<dim3((n + 255) / 256, T), 256, 0, stream>>>(w.yd, ids, wts, gate, T, K, n, 1, resid, out);
    timing_mark(stream, "pf_combine");
    FRT_LAUNCHED("prefill combine");
    return kOk;
}

// expose the dispatch alone (tests compare the permutation with the oracle)
int pf_dispatch(const int32_t* ids, int T, int K, int E, int32_t* bounds, int32_t* tok_of, int32_t* slot_of, void* ws,
                size_t ws_bytes, hipStream_t stream) {
    if (T < 1 || K < 1 || E < 1 || E > 4096) return set_error(kErrShape, "dispatch: T=%d K=%d E=%d", T, K, E);
    const int nchunk = (T * K + kChunk - 1) / kChunk;
    const size_t need = up256(size_t(nchunk) * E * 4) + up256(size_t(pf_max_tiles(T * K, E)) * 8) + 256;
    if (ws_bytes < need) return set_error(kErrWorkspace, "dispatch: workspace %zu < %zu", ws_bytes, need);
    uint8_t* p = static_cast<uint8_t*>(ws);
    int32_t* cnt = reinterpret_cast<int32_t*>(p);
    p += up256(size_t(nchunk) * E * 4);
    int2* tiles = reinterpret_cast<int2*>(p);
    p += up256(size_t(pf_max_tiles(T * K, E)) * 8);
    int32_t* n_tiles = reinterpret_cast<int32_t*>(p);
    int id_bits = 1;
    while ((1 << id_bits) < E) ++id_bits;
    k_pf_hist<<<nchunk, 256, size_t(E) * 4, stream>>>(ids, T * K, E, cnt);
    k_pf_scan<<<1, 1024, 0, stream>>>(cnt, nchunk, E, T, K, 0, bounds, tiles, n_tiles);
    k_pf_place<<<nchunk, 64, size_t(E) * 4, stream>>>(ids, T * K, K, E, id_bits, cnt, tok_of, slot_of);
    FRT_LAUNCHED("dispatch");
    return kOk;
}
size_t pf_dispatch_ws_bytes(int T, int K, int E) {
    const int nchunk = (T * K + kChunk - 1) / kChunk;
    return up256(size_t(nchunk) * E * 4) + up256(size_t(pf_max_tiles(T * K, E)) * 8) + 256;
}

}  // namespace frt
