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

__device__ __forceinline__ int lane_xor16(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? int(r[0]) : int(r[1]);
}
__device__ __forceinline__ int lane_xor32(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? int(r[0]) : int(r[1]);
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

// ---------------------------------------------------------------- grouped GEMMs (gate + up, down)
//
// Weights enter the MFMA exactly: (q - 1) * d_w in fp16, dequantized in registers from the code
// dwords. Activations a = code * d (Q8_0: up to 18 significant bits) enter in NP fp16 parts:
//   NP = 2 (gate/up): hi = fp16(a), lo = fp16(a - hi), so that A * hi + A * lo = A * a exactly; each
//          32-deep MFMA step is issued for both parts into one fp32 accumulator (gfx950's MFMA keeps
//          fp16 subnormals, which the lo parts often are). Exactness here matters because h is
//          requantized to Q8_0 after SwiGLU.
//   NP = 1 (down): fp16(a), 2^-12 relative per element, with no requantization after it.
// No per-block scaling on the VALU either way.
//
// Workgroup: 512 threads (8 waves), 64 tokens x 512 A rows, K in stages of 128 through two LDS
// buffers (the next stage is loaded into registers while the current one is multiplied). Each wave
// owns 4 A tiles of 16 rows and all 4 token tiles, so every activation fragment read from LDS feeds
// 4 NP MFMAs.
//   gate+up: A rows 0..255 are gate rows f0 + 0..255, A rows 256..511 the same up rows; wave w owns
//            ff rows f0 + 32 w .. +31 (gate and up). Epilogue: SwiGLU, Q8_0 of the 32-row block of h
//            (quant/q2_0/moe_cpu.cpp:43-61), h = code * d written as fp16 for the down GEMM.
//   down:    A rows are output rows r0 + 0..511, wave w owns r0 + 64 w .. +63; yd[slot][row] fp32.

constexpr int kKC = 128;          // K per stage
constexpr int kLdB = kKC + 8;     // padded fp16 row of an activation stage

template <int NP>
struct MmStage {
    uint32_t a[512][kKC / 64][4];   // codes: A row, block, dword
    uint32_t sc[512];               // the A row's two fp16 block scales
    _Float16 b[NP][kTN][kLdB];      // activations (perm64 order): [0] fp16(a), [1] a - [0] when NP == 2
};

__device__ __forceinline__ floatx4 mfma_acc(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <bool GATEUP, int NP>
__global__ void __launch_bounds__(512) k_pf_mm(const uint8_t* __restrict__ arena, size_t stride, int E,
                                               const uint8_t* __restrict__ shared_blob, int n, int ff,
                                               const _Float16* __restrict__ bhi, const _Float16* __restrict__ blo,
                                               const int32_t* __restrict__ tok_of, const int32_t* __restrict__ bounds,
                                               const int2* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                               _Float16* __restrict__ hout,
                                               float* __restrict__ yd, const int32_t* __restrict__ slot_of) {
    if (int(blockIdx.y) >= *n_tiles) return;
    extern __shared__ __align__(16) uint8_t smem[];
    MmStage<NP>* st = reinterpret_cast<MmStage<NP>*>(smem);
    __shared__ int sTok[kTN];
    const int2 tile = tiles[blockIdx.y];
    const int grp = tile.x;
    const int row0 = bounds[grp] + tile.y;
    const int cnt = min(kTN, bounds[grp + 1] - row0);
    const uint8_t* blob = grp < E ? arena + size_t(grp) * stride : shared_blob;
    const int Kd = GATEUP ? n : ff;            // contraction length
    const int nbk = Kd / kBlock;               // weight blocks per A row
    const int rows_total = GATEUP ? ff : n;    // rows of each A matrix
    const size_t mb = mat_bytes(ff, n);
    const uint8_t* m0 = GATEUP ? blob : blob + 2 * mb;      // gate (or down)
    const uint8_t* m1 = blob + mb;                          // up
    const int rbase = blockIdx.x * (GATEUP ? 256 : 512);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid < kTN) sTok[tid] = tid < cnt ? (GATEUP ? tok_of[row0 + tid] : row0 + tid) : -1;
    __syncthreads();

    // the A row `ar` of the tile: matrix and row index
    auto arow = [&](int ar, const uint8_t*& m, int& r) {
        if (GATEUP) {
            m = ar < 256 ? m0 : m1;
            r = rbase + (ar & 255);
        } else {
            m = m0;
            r = rbase + ar;
        }
    };
    uint4 ra[2];
    uint32_t rs;
    uint4 rb[2 * NP];
    auto load = [&](int k0) {
        const int b0 = k0 / kBlock;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int idx = p * 512 + tid, ar = idx >> 1, blk = idx & 1;
            const uint8_t* m;
            int r;
            arow(ar, m, r);
            ra[p] = r < rows_total ? *reinterpret_cast<const uint4*>(m + (size_t(r) * nbk + b0 + blk) * 16)
                                   : make_uint4(0, 0, 0, 0);
        }
        {
            const uint8_t* m;
            int r;
            arow(tid, m, r);
            const uint32_t* sc = reinterpret_cast<const uint32_t*>(m + size_t(rows_total) * nbk * 16 + (size_t(r) * nbk + b0) * 2);
            rs = r < rows_total ? *sc : 0u;
        }
#pragma unroll
        for (int p = 0; p < 2 * NP; ++p) {
            const int idx = p * 512 + tid, which = idx >> 10, rem = idx & 1023, j = rem >> 4, q = rem & 15;
            const int t = sTok[j];
            const _Float16* src = which ? blo : bhi;
            rb[p] = t >= 0 ? *reinterpret_cast<const uint4*>(src + size_t(t) * Kd + k0 + q * 8) : make_uint4(0, 0, 0, 0);
        }
    };
    auto store = [&](MmStage<NP>& S) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int idx = p * 512 + tid, ar = idx >> 1, blk = idx & 1;
            *reinterpret_cast<uint4*>(&S.a[ar][blk][0]) = ra[p];
        }
        S.sc[tid] = rs;
#pragma unroll
        for (int p = 0; p < 2 * NP; ++p) {
            const int idx = p * 512 + tid, which = idx >> 10, rem = idx & 1023, j = rem >> 4, q = rem & 15;
            *reinterpret_cast<uint4*>(&S.b[which][j][q * 8]) = rb[p];
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const int li = lane & 15, lg = lane >> 4;
    int art[4];   // this lane's A row in the tile for each of its 4 A tiles
#pragma unroll
    for (int i = 0; i < 4; ++i)
        art[i] = GATEUP ? ((i < 2 ? 0 : 256) + 32 * wave + 16 * (i & 1) + li) : (64 * wave + 16 * i + li);

    const int nstage = Kd / kKC;
    load(0);
    store(st[0]);
    __syncthreads();
    for (int sI = 0; sI < nstage; ++sI) {
        MmStage<NP>& S = st[sI & 1];
        if (sI + 1 < nstage) load((sI + 1) * kKC);
#pragma unroll
        for (int bb = 0; bb < kKC / 64; ++bb) {
            uint32_t cw[4];
            _Float16 dw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                cw[i] = S.a[art[i]][bb][lg];
                dw[i] = __builtin_bit_cast(_Float16, uint16_t(S.sc[art[i]] >> (16 * bb)));
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                half8 av[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) av[i] = dequant8(cw[i], h, dw[i]);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if (c * 16 >= cnt) break;   // token columns past the group's end (ragged tiles)
                    const int col = c * 16 + li, off = bb * 64 + h * 32 + lg * 8;
#pragma unroll
                    for (int part = 0; part < NP; ++part) {
                        const half8 bv = *reinterpret_cast<const half8*>(&S.b[part][col][off]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i][c] = mfma_acc(av[i], bv, acc[i][c]);
                    }
                }
            }
        }
        if (sI + 1 < nstage) {
            store(st[(sI + 1) & 1]);
            __syncthreads();
        }
    }

    if constexpr (GATEUP) {
        // lane: token col c*16 + li; ff rows f = rbase + 32 wave + 16 i + 4 lg + j (i = 0, 1) for gate
        // (acc[i]) and up (acc[2 + i]). The 32 rows of the wave are one Q8_0 block of h.
        const int fbase = rbase + 32 * wave;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = c * 16 + li;
            float hv[2][4];
            float am = 0.0f;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hv[i][j] = silu_mul(acc[i][c][j], acc[2 + i][c][j]);
                    am = fmaxf(am, fabsf(hv[i][j]));
                }
            am = fmaxf(am, __builtin_bit_cast(float, lane_xor16(__builtin_bit_cast(int, am))));
            am = fmaxf(am, __builtin_bit_cast(float, lane_xor32(__builtin_bit_cast(int, am))));
            const float d = q8_scale(am);
            const float id = q8_inv(d);
            const float dr = f16_round(d);
            if (col < cnt && fbase < ff) {
                const size_t row = size_t(row0 + col);
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int f = fbase + 16 * i + 4 * lg + j;
                        const float a = float(q8_code(hv[i][j], id)) * dr;
                        const size_t pos = row * ff + (f & ~63) + perm64_pos(f & 63);
                        hout[pos] = _Float16(a);   // h for the down GEMM, one fp16 part
                    }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = c * 16 + li;
            if (col >= cnt) continue;
            const size_t slot = size_t(slot_of[row0 + col]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = rbase + 64 * wave + 16 * i + 4 * lg;
                if (r < n) *reinterpret_cast<float4*>(yd + slot * n + r) = make_float4(acc[i][c][0], acc[i][c][1], acc[i][c][2], acc[i][c][3]);
            }
        }
    }
}

// ---------------------------------------------------------------- combine

// out[t][i] = sum over the token's K slots in ascending expert id of w * yd (+ shared * sigmoid(g));
// grid (ceil(n / 1024), T), 4 consecutive outputs per thread
template <typename InT>
__global__ void __launch_bounds__(256) k_pf_combine(const InT* __restrict__ yd, const int32_t* __restrict__ ids,
                                                    const float* __restrict__ wts, const float* __restrict__ gate, int T,
                                                    int K, int n, int shared, const float* __restrict__ resid,
                                                    float* __restrict__ out) {
    __shared__ int order[32];
    const int t = blockIdx.y;
    if (threadIdx.x < K) {   // rank of slot k by expert id (the ids of one token are distinct)
        const int e = ids[t * K + threadIdx.x];
        int r = 0;
        for (int k = 0; k < K; ++k) r += ids[t * K + k] < e ? 1 : 0;
        order[r] = threadIdx.x;
    }
    __syncthreads();
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= n) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int r = 0; r < K; ++r) {
        const int k = order[r];
        const float w = wts[t * K + k];
        const InT* src = yd + (size_t(t) * K + k) * n + i;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float p = w * float(src[q]);
            acc[q] = acc[q] + p;
        }
    }
    float o[4] = {acc[0], acc[1], acc[2], acc[3]};
    if (shared) {
        const float g = 1.0f / (1.0f + expf(-gate[t]));
        const InT* src = yd + (size_t(T) * K + t) * n + i;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float p = float(src[q]) * g;
            o[q] = acc[q] + p;
        }
    }
    if (resid)
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = resid[size_t(t) * n + i + q] + o[q];
    *reinterpret_cast<float4*>(out + size_t(t) * n + i) = make_float4(o[0], o[1], o[2], o[3]);
}

// fp32 -> bf16 (round to nearest even), 4 per thread (count % 4 == 0)
__global__ void k_to_bf16(const float* __restrict__ src, __hip_bfloat16* __restrict__ dst, size_t count) {
    const size_t i = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
    if (i >= count) return;
    const float4 v = *reinterpret_cast<const float4*>(src + i);
    dst[i] = __float2bfloat16(v.x);
    dst[i + 1] = __float2bfloat16(v.y);
    dst[i + 2] = __float2bfloat16(v.z);
    dst[i + 3] = __float2bfloat16(v.w);
}

}  // namespace

// ---------------------------------------------------------------- host side

struct PfWs {
    int32_t *cnt, *bounds, *tok_of, *slot_of, *n_tiles;
    int2* tiles;
    _Float16* xhi;
    _Float16* xlo;
    _Float16* hhi;
    float* yd;   // fp32 per-slot outputs when the caller does not receive them as fp32
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
    w.xhi = reinterpret_cast<_Float16*>(take(size_t(T) * n * 2));
    w.xlo = reinterpret_cast<_Float16*>(take(size_t(T) * n * 2));
    w.hhi = reinterpret_cast<_Float16*>(take(size_t(S) * ff * 2));
    w.yd = own_yd ? reinterpret_cast<float*>(take(size_t(S) * n * 4)) : nullptr;
    w.bytes = size_t(p - static_cast<uint8_t*>(base));
    return w;
}

size_t pf_workspace_bytes(int T, int K, int n, int ff, int E, bool shared, bool own_yd) {
    return pf_carve(nullptr, T, K, n, ff, E, shared, own_yd).bytes + 256;
}

int quantize_q8(const float* x, int rows, int n, int8_t* xq, float* xd, _Float16* xhi, _Float16* xlo,
                hipStream_t stream);

int pf_check(int T, int K, int n, int ff, int E) {
    if (T < 1 || K < 1 || K > 32 || E < 1 || E > 4096 || K > E) return set_error(kErrShape, "prefill: T=%d K=%d E=%d", T, K, E);
    if (n % 256 || ff % 128 || n < 256 || ff < 128)
        return set_error(kErrShape, "prefill: n=%d ff=%d (n a multiple of 256, ff of 128)", n, ff);
    return kOk;
}

template <bool GATEUP, int NP>
static int pf_mm_attr() {
    static bool done = false;   // per process; the attribute is a property of the kernel
    if (!done) {
        FRT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_mm<GATEUP, NP>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(2 * sizeof(MmStage<NP>))));
        done = true;
    }
    return kOk;
}

// The two grouped GEMMs. gate/up reads x as exact hi/lo pairs: h is requantized to Q8_0 after
// SwiGLU, and an fp16 rounding of x (2^-12 relative) moves enough h values across a code boundary
// to be seen at the output. down reads h as single fp16 values (2^-12 relative per element,
// summed with no requantization after it).
static int pf_expert_gemms(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff,
                           const PfWs& w, int mt, float* ydf, hipStream_t stream) {
    if (int rc = pf_mm_attr<true, 2>()) return rc;
    if (int rc = pf_mm_attr<false, 1>()) return rc;
    k_pf_mm<true, 2><<<dim3((ff + 255) / 256, mt), 512, 2 * sizeof(MmStage<2>), stream>>>(
        arena, stride, E, shared_blob, n, ff, w.xhi, w.xlo, w.tok_of, w.bounds, w.tiles, w.n_tiles, w.hhi, nullptr,
        nullptr);
    timing_mark(stream, "pf_gateup");
    k_pf_mm<false, 1><<<dim3((n + 511) / 512, mt), 512, 2 * sizeof(MmStage<1>), stream>>>(
        arena, stride, E, shared_blob, n, ff, w.hhi, nullptr, w.tok_of, w.bounds, w.tiles, w.n_tiles, nullptr, ydf,
        w.slot_of);
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
    if (int rc = quantize_q8(x, T, n, nullptr, nullptr, w.xhi, w.xlo, stream)) return rc;
    timing_mark(stream, "pf_quant_x");
    k_pf_hist<<<nchunk, 256, size_t(E) * 4, stream>>>(ids, T * K, E, w.cnt);
    k_pf_scan<<<1, 1024, 0, stream>>>(w.cnt, nchunk, E, T, K, shared ? 1 : 0, w.bounds, w.tiles, w.n_tiles);
    k_pf_place<<<nchunk, 64, size_t(E) * 4, stream>>>(ids, T * K, K, E, id_bits, w.cnt, w.tok_of, w.slot_of);
    if (shared) k_pf_place_shared<<<(T + 255) / 256, 256, 0, stream>>>(T, K, w.tok_of, w.slot_of);
    timing_mark(stream, "pf_dispatch");
    const int mt = pf_max_tiles(S, G);
    float* ydf = yd_kind == 1 ? w.yd : static_cast<float*>(yd);
    if (int rc = pf_expert_gemms(arena, stride, E, shared_blob, n, ff, w, mt, ydf, stream)) return rc;
    if (yd_kind == 1) {
        const size_t cntv = size_t(S) * n;
        k_to_bf16<<<unsigned((cntv / 4 + 255) / 256), 256, 0, stream>>>(ydf, static_cast<__hip_bfloat16*>(yd), cntv);
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
    const PfWs w = pf_carve(ws, T, K, n, ff, E, false, yd_bf16 != 0);
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
    k_pf_combine<float><<<dim3((n + 1023) / 1024, T), 256, 0, stream>>>(w.yd, ids, wts, gate, T, K, n, 1, resid, out);
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
