// Prefill MoE: routed (token, slot) pairs sorted by expert, then grouped GEMMs on fp16 MFMA
// (kernels/cuda/moe_q2.cu:514-548 is the reference's int8 counterpart).
//
// Dispatch (moe_q2.cu:83-168 semantics: a stable sort of slots s = t*K + k by ids[s]):
//   k_pf_hist   per chunk of 256 slots, an LDS histogram of experts (integer atomics only)
//   k_pf_scan   one workgroup: per-expert column prefix over chunks, bounds, the tile list
//   k_pf_place  one wave per chunk walks its slots in order, 64 at a time; each lane's rank among
//               equal experts in the batch comes from ballots (a wave64 match-any), so the
//               placement is stable and needs no atomics.
//   The shared expert, when present, is group E holding every token in order (rows T*K + t, written
//   by the workgroups of k_pf_place past the chunks).
//
// GEMMs (k_pf_gemm, below): Q2_0 weights dequantized exactly to fp16 in registers, activations
// as exact fp16 (hi, lo) pairs (gate/up) or fp16 (down), fp32 accumulation on MFMA; tiles of 64
// tokens of one group; the gate/up epilogue applies SwiGLU and the Q8_0 quantization of h.
//   k_pf_combine out[t] = sum_k (in expert order) w * yd[t*K+k] + yd[shared t] * sigmoid(gate)
#include "common.hpp"

#include <hip/hip_bf16.h>

#include <type_traits>

namespace frt {

constexpr int kTN = 64;        // tokens per GEMM tile
constexpr int kChunk = 256;    // slots per dispatch chunk (one wave of k_pf_place walks one)

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

// Per expert (a wave each): cnt[b][e] becomes the exclusive prefix over the chunks b' < b (the
// chunk's first row within the expert's group), rows[e] the group's size. Lane l takes the chunks
// l P .. l P + P - 1 in order; the lanes' sums are scanned across the wave.
__global__ void __launch_bounds__(256) k_pf_colscan(int32_t* __restrict__ cnt, int nchunk, int E,
                                                    int32_t* __restrict__ rows) {
    const int e = int(blockIdx.x) * 4 + int(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (e >= E) return;   // whole waves
    const int P = (nchunk + 63) / 64, b0 = lane * P, b1 = min(nchunk, b0 + P);
    int sum = 0;
    for (int b = b0; b < b1; ++b) sum += cnt[size_t(b) * E + e];
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    int run = incl - sum;
    for (int b = b0; b < b1; ++b) {
        const int v = cnt[size_t(b) * E + e];
        cnt[size_t(b) * E + e] = run;
        run += v;
    }
    if (lane == 63) rows[e] = incl;
}

// Exclusive prefix sums over the workgroup of N ints per thread at once (and the totals): a shuffle
// scan within each wave, then wave 0 scans the wave totals in parallel. ws: (nwaves + 1) * N ints.
template <int N>
__device__ __forceinline__ void block_excl_scan_v(const int (&v)[N], int (&r)[N], int (&total)[N], int* ws) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int incl[N];
#pragma unroll
    for (int i = 0; i < N; ++i) incl[i] = v[i];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int y = __shfl_up(incl[i], o, 64);
            if (lane >= o) incl[i] += y;
        }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < N; ++i) ws[wave * N + i] = incl[i];
    __syncthreads();
    if (wave == 0) {   // the wave totals: lane w < nw holds wave w's, scanned across the lanes
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int x = lane < nw ? ws[lane * N + i] : 0;
            int c = x;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const int y = __shfl_up(c, o, 64);
                if (lane >= o) c += y;
            }
            if (lane < nw) ws[lane * N + i] = c - x;
            if (lane == nw - 1) ws[nw * N + i] = c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        r[i] = ws[wave * N + i] + incl[i] - v[i];
        total[i] = ws[nw * N + i];
    }
    __syncthreads();
}

// 1024 threads. bounds[e] holds each group's rows (k_pf_colscan) and becomes its first row.
// Tiles are listed longest first (4 token columns of 16, then 3, 2, 1; by expert within a class),
// so that the grouped GEMMs start the long tiles first and finish on short ones.
__device__ __forceinline__ int tile_class(int rows) { return (rows + 15) / 16; }   // 1..4

// The body of k_pf_scan for a 1024-thread workgroup: s_rows[e] (LDS) holds group e's rows on entry
// and its first row on exit; bounds[e] gets the same first rows (bounds[E] = T K, bounds[E + 1] =
// T K + T with the shared group), tiles and n_tiles the tile list.
__device__ void pf_scan_body(int* s_rows, int E, int T, int shared, int32_t* __restrict__ bounds,
                             int2* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
    __shared__ int ws[17 * 5];
    static_assert(1024 / 64 <= 16, "the wave-total scan covers 16 waves");
    // tiles of each class of group e (rows c): c / 64 full tiles (class 4) and one of class (c % 64)
    auto count = [&](int c, int (&n)[5]) {
        n[1] = n[2] = n[3] = n[4] = 0;
        n[4] = c / kTN;
        if (c % kTN) ++n[tile_class(c % kTN)];
    };
    // pass 1: tiles per class over all groups (the shared group E included)
    int total[5] = {0, 0, 0, 0, 0};
    for (int e0 = 0; e0 < E; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        int n[5];
        count(e < E ? s_rows[e] : 0, n);
        const int v[4] = {n[1], n[2], n[3], n[4]};
        int r[4], tot[4];
        block_excl_scan_v<4>(v, r, tot, ws);
        for (int k = 1; k <= 4; ++k) total[k] += tot[k - 1];
    }
    int sh[5] = {0, 0, 0, 0, 0};
    if (shared) {
        count(T, sh);
        for (int k = 1; k <= 4; ++k) total[k] += sh[k];
    }
    int base[5];   // first tile of each class
    base[4] = 0;
    for (int k = 3; k >= 1; --k) base[k] = base[k + 1] + total[k + 1];
    // pass 2: bounds, chunk offsets for k_pf_place, and the tiles
    int run_rows = 0;
    for (int e0 = 0; e0 < E; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        const int c = e < E ? s_rows[e] : 0;   // (each thread reads and then writes only its own groups')
        int n[5], at[5];
        count(c, n);
        const int v[5] = {c, n[1], n[2], n[3], n[4]};
        int r[5], tot[5];
        block_excl_scan_v<5>(v, r, tot, ws);
        const int off = r[0] + run_rows, tot_rows = tot[0];
        for (int k = 1; k <= 4; ++k) {
            at[k] = r[k] + base[k];
            base[k] += tot[k];
        }
        if (e < E) {
            bounds[e] = off;
            s_rows[e] = off;
            for (int i = 0; i < c / kTN; ++i) tiles[at[4] + i] = make_int2(e, i * kTN);
            if (c % kTN) {
                const int k = tile_class(c % kTN);
                tiles[at[k] + (k == 4 ? n[4] - 1 : 0)] = make_int2(e, (c / kTN) * kTN);
            }
        }
        run_rows += tot_rows;
    }
    if (threadIdx.x == 0) {
        bounds[E] = run_rows;   // = T * K
        if (shared) {
            bounds[E + 1] = run_rows + T;
            for (int i = 0; i < T / kTN; ++i) tiles[base[4] + i] = make_int2(E, i * kTN);
            if (T % kTN) {
                const int k = tile_class(T % kTN);
                tiles[base[k] + (k == 4 ? sh[4] - 1 : 0)] = make_int2(E, (T / kTN) * kTN);
            }
        }
        n_tiles[0] = total[1] + total[2] + total[3] + total[4];
        n_tiles[1] = total[2] + total[3] + total[4];   // the one-column tiles come last
    }
    __syncthreads();
}

__global__ void __launch_bounds__(1024) k_pf_scan(int E, int T, int shared, int32_t* __restrict__ bounds,
                                                  int2* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
    __shared__ int s_rows[4096];   // (E <= 4096)
    for (int e = threadIdx.x; e < E; e += blockDim.x) s_rows[e] = bounds[e];   // (k_pf_colscan's group sizes)
    __syncthreads();
    pf_scan_body(s_rows, E, T, shared, bounds, tiles, n_tiles);
}

// one wave per chunk; stable ranks from a ballot match-any over the expert id bits
__global__ void __launch_bounds__(64) k_pf_place(const int32_t* __restrict__ ids, int S, int K, int E, int id_bits,
                                                 const int32_t* __restrict__ cnt, const int32_t* __restrict__ bounds,
                                                 int32_t* __restrict__ tok_of, int32_t* __restrict__ slot_of, int shared_T) {
    extern __shared__ int32_t next[];
    const int lane = threadIdx.x;
    const int nchunk = (S + kChunk - 1) / kChunk;
    if (int(blockIdx.x) >= nchunk) {   // the workgroups past the chunks: the shared group's rows S + t
        const int t = (int(blockIdx.x) - nchunk) * 64 + lane;
        if (t < shared_T) {
            tok_of[S + t] = t;
            slot_of[S + t] = S + t;
        }
        return;
    }
    for (int e = lane; e < E; e += 64) next[e] = bounds[e] + cnt[size_t(blockIdx.x) * E + e];
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

// ---------------------------------------------------------------- grouped GEMMs (gate + up, down)
//
// Operands enter the MFMA exactly, so the products are exact and only the fp32 accumulation rounds:
//   A (weights): (q - 1) * d_w in fp16, dequantized in registers from the code dwords.
//   B (activations a = code * d_a, Q8_0: up to 18 significant bits), in NP fp16 parts:
//     NP = 2 (gate/up): hi = fp16(a), lo = fp16(a - hi); every 32-deep MFMA step is issued for
//            both parts into one fp32 accumulator (gfx950's MFMA keeps the fp16 subnormals that
//            the lo parts can be). Exactness matters here because h is requantized to Q8_0 after
//            SwiGLU: a rounding difference would move h codes across rounding boundaries.
//     NP = 1 (down): fp16(a), 2^-12 relative per element, with no requantization after it.
//   No per-block scaling happens on the VALU.
//
// Dequantization: code k of a weight dword sits at bits 2k, 2k+1. Masked in place (p = 2k mod 8
// within each 16-bit half) and OR'ed with the fp16 bits of M = 2^(10-p), whose ulp is 2^(p-10),
// it reads as M + q exactly; (M + q) - (M + 1) = q - 1 and the product with d_w are exact too.
// Codes 4..7 of each half are shifted down by 8 first. Per pair of weights: one v_and_or_b32,
// one v_pk_add_f16 and one v_pk_mul_f16 (plus one shift per 16 weights).
//
// k_pf_gemm<SMALL>: the gate/up GEMM. A tile's A rows are ff rows f0 .. of gate and the same rows of
// up; wave w owns 32 of them (2 gate + 2 up tiles of 16), so SwiGLU and the Q8_0 of a 32-row block
// of h (quant/q2_0/moe_cpu.cpp:43-61) are lane-local; h = code * d is written as fp16 for the down
// GEMM. Two shapes:
//   SMALL = false: 256 threads (4 waves), 64 tokens x 128 ff rows, activation stages of K = 64 (a
//                  48 KB ring), so two workgroups share a CU and one computes while the other waits
//                  for its loads; the tile classes of 2-4 token columns (one branch-free variant per
//                  column count).
//   SMALL = true:  256 threads, 16 tokens x 128 ff rows, stages of K = 256 in a ring of 2, for the tiles of one
//                  token column (half of them under skewed routing): a quarter of the LDS and of the
//                  registers, so 4 workgroups share a CU.
// Every activation fragment read from LDS feeds 4 MFMAs, every dequantized weight fragment NC NP.
//
// K order (perm256_pos): within each 256-element stretch, MFMA lane group g takes block g of the
// stretch. So the weights go straight from HBM into registers: lane (row i, group g) loads the
// 16-byte code chunk of block g of its row, and the 4 lanes of a row read 64 contiguous bytes (a
// weight row is a separate 512-byte stretch of HBM; one lane per row and 16-byte chunk would make
// every lane a separate cache-line request). Each wave loads only its own rows, one stretch ahead,
// into a second register set.
//
// Activations go through LDS: stages of 64 or 128 K in a ring of 3 slots
// filled by direct global-to-LDS loads (global_load_lds: each lane's 16 bytes land at the wave's LDS
// base + 16 lane, no registers), issued 2 stages ahead; one workgroup barrier per stage. Slot layout:
//   [NP][tokens][cpt chunks of 8 fp16], chunk kc of token j at j * cpt + (kc ^ (j % cpt)), so that the
//   lanes of a 128-bit read phase (one chunk of 8 tokens) hit distinct bank groups.
// Issue order of k_pf_gemm's loads, as stages s of the same pattern: stage s issues the weights of
// stretch s / sps + 1 when s is a stretch's first (s % sps == 0: "A"), then the activations of stage
// s + ahead ("B"). The prologue is the stages s = -max(ahead, sps) .. -1 of that pattern (A of
// stretch 0 at s = -sps; B stage s + ahead for s >= -ahead), so every stage's wait counts the same.
constexpr int gu_mod(int a, int m) { return ((a % m) + m) % m; }
// The vmcnt of stage st's wait: the loads issued after B stage st (at stage st - ahead), by stages
// st - ahead + 1 .. st - 1: ahead - 1 B stages and the A of each stretch's first among them.
constexpr int gu_wait(int h, int ahead, int sps, int kDB, int kDA) {
    int c = (ahead - 1) * kDB;
    for (int d = 1; d < ahead; ++d) c += gu_mod(h - d, sps) == 0 ? kDA : 0;
    return c;
}
// The same count by listing the issues of the prologue and stages 0 .. st - 1 (1 = an A, 2 + s = B
// stage s) and counting what follows B stage st.
constexpr int gu_after_b(int st, int ahead, int sps, int kDB, int kDA) {
    int seq[96] = {};
    int n = 0;
    const int first = -(ahead > sps ? ahead : sps);
    for (int s = first; s < st; ++s) {
        if (gu_mod(s, sps) == 0 && s / sps + 1 >= 0 && s >= -sps) seq[n++] = 1;
        if (s >= -ahead) seq[n++] = 2 + s + ahead;
    }
    int after = 0;
    bool seen = false;
    for (int i = 0; i < n; ++i) {
        if (seen) after += seq[i] == 1 ? kDA : kDB;
        if (seq[i] == 2 + st) seen = true;
    }
    return after;
}
constexpr bool gu_waits_ok(int ahead, int sps, int kDB, int kDA) {
    for (int st = 0; st < 16; ++st)
        if (gu_after_b(st, ahead, sps, kDB, kDA) != gu_wait(gu_mod(st, sps), ahead, sps, kDB, kDA)) return false;
    return true;
}
template <bool SMALL>
struct GuShape {
    static constexpr int threads = 256;
    static constexpr int tokens = SMALL ? 16 : kTN;       // activation rows in LDS
    static constexpr int ff_rows = threads / 2;           // ff rows per workgroup (32 per wave)
    static constexpr int stage_k = SMALL ? 256 : 64;      // K per activation stage
    static constexpr int sps = 256 / stage_k;             // stages per weight stretch
    static constexpr int ksps = stage_k / 32;             // MFMA K-steps per stage
    static constexpr int cpt = stage_k / 8;               // 16-byte chunks per token per stage
    static constexpr int slot_b = tokens * stage_k * 2;   // bytes per part per slot
    static constexpr int stages = SMALL ? 2 : 3;          // activation ring slots
    static constexpr int ahead = stages - 1;              // stages issued ahead
    static constexpr int smem = stages * 2 * slot_b;
    static constexpr int dma = tokens * cpt / threads;    // activation loads per lane per part
    static constexpr int min_waves = SMALL ? 4 : 2;       // per SIMD (SMALL: 4 workgroups per CU)
    static_assert(sps <= 4 && gu_waits_ok(ahead, sps, dma * 2, 8), "the wait counts of k_pf_gemm");
};


typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;
// direct global -> LDS load of 16 bytes per lane to lds_base + 16 lane (lds_base uniform)
__device__ __forceinline__ void ldsdma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)g, (lds_ptr_t)lds_base, 16, 0, 0);
}
// A workgroup barrier that does not wait for outstanding global loads (__syncthreads' release fence
// would wait for all of them, the ring's later stages included): this wave's LDS accesses complete,
// then s_barrier. The wait is the builtin (so the compiler's own wait insertion knows the LDS reads
// before it are complete); the empty asm statements keep memory accesses from moving across.
__device__ __forceinline__ void ring_barrier() {
    __builtin_amdgcn_sched_barrier(0);   // nothing is scheduled across (register math included)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt and expcnt not waited for
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
// s_waitcnt with vmcnt = N (gfx9 encoding; expcnt and lgkmcnt not waited for)
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}
// (x & mask) | bits as one v_and_or_b32 (with literal operands the compiler splits it in two)
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bits));
    return r;
}

// The fp16 bits of 2^(10 - 2m) in both halves, m = 0..3, held in VGPRs
struct DqMagic {
    uint32_t v[4];
};
__device__ __forceinline__ DqMagic dq_magic() {
    DqMagic r;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        r.v[m] = (0x6400u - 0x0800u * m) * 0x00010001u;
        asm volatile("" : "+v"(r.v[m]));
    }
    return r;
}

// The 8 A operand values of K-step h of one weight row's code dword: pass cw for h = 0 and cw >> 8
// for h = 1; dd = the row's block scale in both halves.
__device__ __forceinline__ half8 dequant8(uint32_t c, half2v dd, const DqMagic& mg) {
    half8 a;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const _Float16 off = _Float16(float((1 << (10 - 2 * m)) + 1));
        const half2v offs = {off, off};
        half2v v = __builtin_bit_cast(half2v, and_or(c, 0x00030003u << (2 * m), mg.v[m]));
        v = (v - offs) * dd;
        a[2 * m] = v[0];
        a[2 * m + 1] = v[1];
    }
    return a;
}

__device__ __forceinline__ int lane_xor16(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? int(r[0]) : int(r[1]);
}
__device__ __forceinline__ int lane_xor32(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? int(r[0]) : int(r[1]);
}

__device__ __forceinline__ floatx4 mfma_acc(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }


template <bool SMALL>
__global__ void __launch_bounds__(GuShape<SMALL>::threads, GuShape<SMALL>::min_waves)
k_pf_gemm(const uint8_t* __restrict__ arena, size_t stride, int E, const uint8_t* __restrict__ shared_blob, int n,
          int np, int hblk, int ff, const _Float16* __restrict__ bhi, const _Float16* __restrict__ blo,
          const int32_t* __restrict__ tok_of, const int32_t* __restrict__ bounds, const int2* __restrict__ tiles,
          const int32_t* __restrict__ n_tiles, _Float16* __restrict__ hout) {
    using Sh = GuShape<SMALL>;
    constexpr int NP = 2;
    constexpr int kDB = Sh::dma * NP;   // activation loads per lane per stage
    constexpr int kDA = 8;              // weight loads per lane per stretch (4 code chunks + 4 scales)
    // A 1-D grid of gx ff-slices x tiles (tiles rounded up to a multiple of 8). Workgroup L runs on
    // XCD L % 8, so the slices of a tile are placed 8 apart: they run on the same XCD at about the same
    // time, and the tile's activations come into that XCD's L2 once.
    const int gx = ff / Sh::ff_rows;
    const int ffp = (ff + 255) & ~255;   // h row length
    const int L = blockIdx.x, r8 = L >> 3;
    const int slice = r8 % gx, t = (L & 7) + 8 * (r8 / gx);
    // n_tiles[0]: tiles in all; n_tiles[1]: the first tile of one token column (the list is ordered
    // longest first). The small shape takes those, the other the rest.
    const int ti = SMALL ? n_tiles[1] + t : t;
    if (ti >= (SMALL ? n_tiles[0] : n_tiles[1])) return;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sRow[Sh::tokens];
    const int2 tile = tiles[ti];
    const int grp = tile.x;
    const int row0 = bounds[grp] + tile.y;
    const int cnt = min(Sh::tokens, bounds[grp + 1] - row0);
    const uint8_t* blob = grp < E ? arena + size_t(grp) * stride : shared_blob;
    const int nbk = n / kBlock;   // weight blocks per row
    const size_t mb = mat_bytes(ff, n);
    const int rbase = slice * Sh::ff_rows;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;
    // activation row of each tile token; past the group's end the first repeats (never written)
    if (tid < Sh::tokens) sRow[tid] = tok_of[row0 + min(tid, cnt - 1)];
    __syncthreads();

    // this lane's weight rows: ff row rbase + 32 wave + 16 (i & 1) + li of gate (i < 2) and up;
    // rows past the end load any row and are never stored. aoff = row * nbk: the chunk and scale
    // index of the row's block 0. K runs to np (n rounded up to 512, the activations zero past n):
    // a block past the row's last is read as its last, whose finite products with zeros are 0.
    const uint8_t* const mG = blob;
    const uint8_t* const mU = blob + mb;
    const size_t scale_off = size_t(ff) * nbk * 16;
    uint32_t aoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) aoff[i] = uint32_t(min(rbase + 32 * wave + 16 * i + li, ff - 1)) * nbk;
    struct ARegs {
        uint4 cw[4];
        uint32_t sc[4];
    };
    auto load_a = [&](int q, ARegs& a) {   // stretch q (blocks 4q + lg)
        const int bq = min(4 * q + lg, nbk - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t* m = i < 2 ? mG : mU;
            const size_t o = size_t(aoff[i & 1]) + bq;
            a.cw[i] = gld_u4(m + o * 16);
            a.sc[i] = gld<uint16_t>(m + scale_off + o * 2);
        }
    };
    // this thread's activation chunks of a stage: LDS positions P = threads p + tid (token P / 16)
    uint32_t boff[Sh::dma];   // element offsets (rows * n stays below 2^31)
#pragma unroll
    for (int p = 0; p < Sh::dma; ++p) {
        const int P = Sh::threads * p + tid, j = P / Sh::cpt, kc = (P % Sh::cpt) ^ (j & (Sh::cpt - 1));
        boff[p] = uint32_t(sRow[j]) * np + kc * 8;
    }
    auto issue_b = [&](int st, int slot) {
        uint8_t* b = smem + slot * NP * Sh::slot_b;
#pragma unroll
        for (int p = 0; p < Sh::dma; ++p) {
            ldsdma16(bhi + boff[p] + size_t(st) * Sh::stage_k, b + p * Sh::threads * 16 + wave * 1024);
            ldsdma16(blo + boff[p] + size_t(st) * Sh::stage_k, b + Sh::slot_b + p * Sh::threads * 16 + wave * 1024);
        }
    };
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const DqMagic mg = dq_magic();

    // K-step t of stage st (K-step tt of the stretch whose weights are in a), by token column: column
    // 0's activations are read first, the 4 A fragments dequantized while they land, then each
    // column's MFMAs run while the next column's activations are read (two column buffers).
    auto kstep = [&](auto nc, int st, int t, const ARegs& a, int tt) {
        constexpr int NC = decltype(nc)::value;
        const half8* sb = reinterpret_cast<const half8*>(smem + (st % Sh::stages) * NP * Sh::slot_b);
        auto rd = [&](int c, half8(&b)[NP]) {
            const int j = c * 16 + li, kc = t * 4 + lg;
#pragma unroll
            for (int part = 0; part < NP; ++part) b[part] = sb[part * (Sh::slot_b / 16) + j * Sh::cpt + (kc ^ (j & (Sh::cpt - 1)))];
        };
        half8 b0[NP], b1[NP];
        rd(0, b0);
        half8 av[4];
        const int d = tt >> 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 w = a.cw[i];
            const uint32_t cw = d == 0 ? w.x : d == 1 ? w.y : d == 2 ? w.z : w.w;
            const _Float16 sc = __builtin_bit_cast(_Float16, uint16_t(a.sc[i]));
            av[i] = dequant8((tt & 1) ? cw >> 8 : cw, half2v{sc, sc}, mg);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            half8(&cur)[NP] = (c & 1) ? b1 : b0;
            half8(&nxt)[NP] = (c & 1) ? b0 : b1;
            if (c + 1 < NC) rd(c + 1, nxt);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int part = 0; part < NP; ++part) acc[i][c] = mfma_acc(av[i], cur[part], acc[i][c]);
        }
    };

    // Stage st (K = stage_k st ..) is part h = st % sps of stretch st / sps. Per stage st, after its
    // barrier: A stretch st / sps + 1 (first stage of a stretch, h = 0), then B stage st + ahead (the
    // issue pattern of gu_wait). Waiting for B stage st (vmcnt: the loads issued after it may stay
    // outstanding) covers everything issued before it, A stretch st / sps included. The pattern is
    // the same for every stage: past the end, the last stretch / stage is loaded again (into
    // registers / a slot nothing reads any more), so the wait counts are constants and the
    // compiler's own waits for the weight registers never see a path without later loads (at such
    // a merge it would wait for every load in flight).
    const int nst = np / Sh::stage_k;   // stages
    const int nq = np / 256;            // stretches (even)
    auto run = [&](auto nc) {
        ARegs a0, a1;   // stretches of even / odd index (named, so they stay in registers)
        // the loads of stages -max(ahead, sps) .. -1 of the steady-state pattern below
#pragma unroll
        for (int s = -(Sh::ahead > Sh::sps ? Sh::ahead : Sh::sps); s < 0; ++s) {
            if (gu_mod(s, Sh::sps) == 0 && s >= -Sh::sps) load_a(0, a0);
            if (s >= -Sh::ahead) issue_b(min(s + Sh::ahead, nst - 1), s + Sh::ahead);
        }
        // the two stages of stretch q, whose weights are in cur; the next stretch loads into nxt
        auto stretch = [&](int q, const ARegs& cur, ARegs& nxt) {
#pragma unroll
            for (int h = 0; h < Sh::sps; ++h) {
                const int st = Sh::sps * q + h;
                // loads issued after B stage st (by stages st - ahead + 1 .. st - 1) may stay outstanding
                switch (h) {
                    case 0: wait_vm<gu_wait(0, Sh::ahead, Sh::sps, kDB, kDA)>(); break;
                    case 1: wait_vm<gu_wait(1, Sh::ahead, Sh::sps, kDB, kDA)>(); break;
                    case 2: wait_vm<gu_wait(2, Sh::ahead, Sh::sps, kDB, kDA)>(); break;
                    default: wait_vm<gu_wait(3, Sh::ahead, Sh::sps, kDB, kDA)>(); break;
                }
                ring_barrier();   // stage st is in LDS for every wave; every wave is done with stage st - 1
                if (h == 0) load_a(min(q + 1, nq - 1), nxt);
                issue_b(min(st + Sh::ahead, nst - 1), (st + Sh::ahead) % Sh::stages);   // into stage st - 1's slot
#pragma unroll
                for (int t = 0; t < Sh::ksps; ++t) kstep(nc, st, t, cur, Sh::ksps * h + t);
            }
        };
        for (int q = 0; q < nq; q += 2) {   // nq is even
            stretch(q, a0, a1);
            stretch(q + 1, a1, a0);
        }
    };
    if constexpr (SMALL) {
        run(std::integral_constant<int, 1>{});
    } else {
        switch ((cnt + 15) / 16) {   // token columns with at least one real token (2..4 here)
            case 2: run(std::integral_constant<int, 2>{}); break;
            case 3: run(std::integral_constant<int, 3>{}); break;
            default: run(std::integral_constant<int, 4>{}); break;
        }
    }

    // lane: token column c*16 + li; ff rows f = rbase + 32 wave + 16 i + 4 lg + r (i = 0, 1) for gate
    // (acc[i]) and up (acc[2 + i]). The 32 rows of the wave are one Q8_0 block of h.
    const int fbase = rbase + 32 * wave;
#pragma unroll
    for (int c = 0; c < (SMALL ? 1 : 4); ++c) {
        const int col = c * 16 + li;
        float hv[2][4];
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                hv[i][r] = silu_mul(acc[i][c][r], acc[2 + i][c][r]);
                am = fmaxf(am, fabsf(hv[i][r]));
            }
        am = fmaxf(am, __builtin_bit_cast(float, lane_xor16(__builtin_bit_cast(int, am))));
        am = fmaxf(am, __builtin_bit_cast(float, lane_xor32(__builtin_bit_cast(int, am))));
        if (hblk == 64) {   // ff rows 64 m .. 64 m + 63 are waves 2m' and 2m' + 1 (rbase is a multiple of 128)
            wait_vm<0>();      // the ring's last direct-to-LDS loads (repeats past the end) have landed
            __syncthreads();   // (uniform: hblk is a kernel argument) every wave is past its last LDS read
            float* sam = reinterpret_cast<float*>(smem);
            if (lg == 0) sam[wave * 16 + li] = am;
            __syncthreads();
            am = fmaxf(am, sam[(wave ^ 1) * 16 + li]);
        }
        const float d = q8_scale(am);
        const float id = q8_inv(d);
        const float dr = f16_round(d);
        if (col < cnt && fbase < ff) {
            const size_t row = size_t(row0 + col);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = fbase + 16 * i + 4 * lg + r;
                    const float a = float(q8_code(hv[i][r], id)) * dr;
                    hout[row * ffp + (f & ~255) + perm256_pos(f & 255)] = _Float16(a);
                }
        }
    }
    // h rows are ffp = ff rounded up to 256 long (whole perm256 stretches for the down GEMM); the
    // slice holding the last rows also writes zeros at the pad's positions, so that the down GEMM's
    // products there are 0 (its weights for the pad are any finite values of the row)
    if (ffp > ff && rbase + Sh::ff_rows >= ff) {
        const int np = ffp - ff;   // pad elements per row: f = ff .. ffp - 1
        for (int i = tid; i < cnt * np; i += Sh::threads) {
            const int col = i / np, f = ff + i % np;
            hout[size_t(row0 + col) * ffp + (f & ~255) + perm256_pos(f & 255)] = _Float16(0.0f);
        }
    }
}

// k_pf_down: the down GEMM, one workgroup (256 threads) per tile. The tile's activations (h of 64
// dispatched rows, all of K = ffp = ff rounded up to 256, perm256 order, zeros in the pad) are loaded
// into LDS once (64 tokens x ffp fp16; chunk kc of token j at j * ffp / 8 + (kc ^ (j & 15))), then
// the workgroup walks all n output rows in blocks
// of 256 (wave w: rows 64 w + 16 i + li of the block), streaming the weights straight into
// registers with three stretches of lookahead (four register sets). No barrier after the
// activation load: each wave reads only its own weights. Two workgroups share a CU (64 KB of LDS
// each for ff = 512), so one computes while the other waits for loads. NQ = ffp / 256 stretches per
// row block; a weight block past the row's last (the pad) is read as the row's last block, whose
// finite products with the pad's zeros are 0. TAIL: the stretch count is not a multiple of 4, and
// the last round of 4 steps has steps past the end (loads repeated, no products).
// 4 consecutive per-slot outputs as float, fp16 or bf16 (round to nearest even)
__device__ __forceinline__ void store4(float* p, floatx4 v) { *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]); }
__device__ __forceinline__ void store4(_Float16* p, floatx4 v) {
    typedef _Float16 half4v __attribute__((ext_vector_type(4)));
    const half4v h = {_Float16(v[0]), _Float16(v[1]), _Float16(v[2]), _Float16(v[3])};
    *reinterpret_cast<half4v*>(p) = h;
}
// (chunked down: fp32 only; the chunks run one after another on the stream)
__device__ __forceinline__ void add4(float* p, floatx4 v) {
    float4 o = *reinterpret_cast<float4*>(p);
    o.x += v[0];
    o.y += v[1];
    o.z += v[2];
    o.w += v[3];
    *reinterpret_cast<float4*>(p) = o;
}
template <typename T>
__device__ __forceinline__ void add4(T*, floatx4) {}
__device__ __forceinline__ void store4(__hip_bfloat16* p, floatx4 v) {
    p[0] = __float2bfloat16(v[0]);
    p[1] = __float2bfloat16(v[1]);
    p[2] = __float2bfloat16(v[2]);
    p[3] = __float2bfloat16(v[3]);
}

// ff above 1024 runs in chunks of K = 1024 (the tile's activations of one chunk in LDS): chunk k0 .. k0
// + 256 NQ - 1 of h (rows hstride long) against weight blocks k0 / 64 .. of each row, the chunk's
// products added to yd (fp32) after the first chunk (accumulate).
// SMALL: the one-column tiles (16 tokens; the list's n_tiles[1] .. n_tiles[0] - 1) with a quarter of
// the LDS and at most 168 registers, so 3 workgroups share a CU; otherwise the tiles before them
// (2-4 columns). Measured on configs[3]: the layer 542 -> 522 us against one kernel for all tiles.
template <int NQ, bool TAIL, typename OutT, bool SMALL>
__global__ void __launch_bounds__(256, SMALL ? 3 : 2) k_pf_down(const uint8_t* __restrict__ arena, size_t stride, int E,
                                                 const uint8_t* __restrict__ shared_blob, int n, int ff,
                                                 const _Float16* __restrict__ h, const int32_t* __restrict__ bounds,
                                                 const int2* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                 OutT* __restrict__ yd, const int32_t* __restrict__ slot_of, int k0,
                                                 int hstride, int accumulate) {
    constexpr int ffp = NQ * 256;      // the chunk's h length
    const int nbk = ff / kBlock;       // weight blocks per row
    const int b0 = k0 / kBlock;        // the chunk's first weight block
    const int nbc = min(nbk - b0, ffp / kBlock);   // weight blocks of the chunk
    constexpr int cpt = ffp / 8;       // 16-byte activation chunks per token
    constexpr int TN = SMALL ? 16 : kTN;   // tokens per tile
    constexpr int MC = TN / 16;              // token columns at most
    constexpr int kDB = TN * cpt / 256;      // activation loads per lane
    static_assert(TN * cpt % 256 == 0, "whole activation loads per lane");
    const int ti = SMALL ? n_tiles[1] + int(blockIdx.y) : int(blockIdx.y);
    if (ti >= n_tiles[SMALL ? 0 : 1]) return;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sRow[TN];
    const int2 tile = tiles[ti];
    const int grp = tile.x;
    const int row0 = bounds[grp] + tile.y;
    const int cnt = min(TN, bounds[grp + 1] - row0);
    const uint8_t* blob = grp < E ? arena + size_t(grp) * stride : shared_blob;
    const uint8_t* const md = blob + 2 * mat_bytes(ff, n);   // down [n][ff]
    const size_t scale_off = size_t(n) * nbk * 16;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;
    if (tid < TN) sRow[tid] = row0 + min(tid, cnt - 1);   // past the group's end: repeat a row
    __syncthreads();
#pragma unroll
    for (int p = 0; p < kDB; ++p) {
        const int P = 256 * p + tid, j = P / cpt, kc = (P % cpt) ^ (j & 15);
        ldsdma16(h + size_t(sRow[j]) * hstride + k0 + kc * 8, smem + P * 16 - lane * 16);
    }

    uint32_t aoff[4];   // this lane's row in its row block, for tile i
#pragma unroll
    for (int i = 0; i < 4; ++i) aoff[i] = uint32_t(64 * wave + 16 * i + li);
    struct ARegs {
        uint4 cw[4];
        uint32_t sc[4];
    };
    const int nsx = ((n + 255) / 256) * NQ;   // stretches in all (a multiple of 4 unless TAIL)
    // stretch s: row block s / NQ, blocks 4 (s % NQ) + lg; rows past n (a last block of 128 rows)
    // read row n - 1 and are never stored
    auto load_a = [&](int s, ARegs& a) {
        const int rb = s / NQ;
        const uint32_t blk = b0 + min(4 * (s % NQ) + lg, nbc - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t o = size_t(min(rb * 256 + int(aoff[i]), n - 1)) * nbk + blk;
            a.cw[i] = gld_u4(md + o * 16);
            a.sc[i] = gld<uint16_t>(md + scale_off + o * 2);
        }
    };
    const DqMagic mg = dq_magic();

    size_t yslot[MC];   // yd row of this lane's token column c (loaded before the weight stream)
#pragma unroll
    for (int c = 0; c < MC; ++c) yslot[c] = size_t(slot_of[row0 + min(c * 16 + li, cnt - 1)]) * n;
    auto run = [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        ARegs a0, a1, a2, a3;
        floatx4 acc[4][NC];
        load_a(0, a0);
        load_a(min(1, nsx - 1), a1);
        load_a(min(2, nsx - 1), a2);
        wait_vm<3 * 8>();   // the activations (issued first) are in LDS for this wave ...
        __syncthreads();    // ... and for every wave
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        const half8* sb = reinterpret_cast<const half8*>(smem);
        // stretch s with weights in cur; the stretch three ahead loads into nxt (the last one again
        // past the end, so every stretch has the same loads in flight)
        auto step = [&](int s, int q, const ARegs& cur, ARegs& nxt) {
            load_a(min(s + 3, nsx - 1), nxt);
            if (TAIL && s >= nsx) return;   // past the end (uniform)
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                half8 bv[4];
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const int j = c * 16 + li, kc = (q * 8 + tt) * 4 + lg;
                    bv[c] = sb[j * cpt + (kc ^ (j & 15))];
                }
                const int d = tt >> 1;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 w = cur.cw[i];
                    const uint32_t cw = d == 0 ? w.x : d == 1 ? w.y : d == 2 ? w.z : w.w;
                    const _Float16 sc = __builtin_bit_cast(_Float16, uint16_t(cur.sc[i]));
                    const half8 av = dequant8((tt & 1) ? cw >> 8 : cw, half2v{sc, sc}, mg);
#pragma unroll
                    for (int c = 0; c < NC; ++c) acc[i][c] = mfma_acc(av, bv[c], acc[i][c]);
                }
            }
            if (q == NQ - 1) {   // row block s / NQ done: yd[slot][row], then a fresh block
                const int rb = s / NQ;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    if (c * 16 + li < cnt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int r = rb * 256 + 64 * wave + 16 * i + 4 * lg;
                            if (r < n) {   // (n % 4 == 0)
                                if (accumulate) add4(yd + yslot[c] + r, acc[i][c]);
                                else store4(yd + yslot[c] + r, acc[i][c]);
                            }
                        }
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
        };
        // the stretch's place in its row block: a constant per unrolled step when NQ divides 4
        auto qof = [&](int s, int i) { return 4 % NQ == 0 ? i % NQ : s % NQ; };
        for (int s = 0; s < nsx; s += 4) {
            step(s, qof(s, 0), a0, a3);
            step(s + 1, qof(s + 1, 1), a1, a0);
            step(s + 2, qof(s + 2, 2), a2, a1);
            step(s + 3, qof(s + 3, 3), a3, a2);
        }
    };
    if constexpr (SMALL) {
        run(std::integral_constant<int, 1>{});
    } else {
        switch ((cnt + 15) / 16) {   // token columns with at least one real token (2..4 here)
            case 2: run(std::integral_constant<int, 2>{}); break;
            case 3: run(std::integral_constant<int, 3>{}); break;
            default: run(std::integral_constant<int, 4>{}); break;
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

}  // namespace

// ---------------------------------------------------------------- host side

struct PfWs {
    int32_t *cnt, *bounds, *tok_of, *slot_of, *n_tiles;
    int2* tiles;
    _Float16 *xhi, *xlo;   // x = code * d as an exact fp16 pair, perm256 order [T][n]
    _Float16* h16;         // h = code * d as fp16, perm256 order [S][ffp], ffp = ff rounded up to 256
    _Float16* yd;   // fp16 per-slot outputs of a whole layer (combined by k_pf_combine)
    size_t bytes;
};

static int pf_max_tiles(int S, int G) { return (S + kTN - 1) / kTN + G; }
// the gate/up GEMM's K extent: n rounded up to whole pairs of 256-element stretches
static int pf_np(int n) { return (n + 511) & ~511; }

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
    w.n_tiles = reinterpret_cast<int32_t*>(take(8));   // [0] tiles, [1] first tile of one column
    w.tiles = reinterpret_cast<int2*>(take(size_t(pf_max_tiles(S, G)) * 8));
    w.xhi = reinterpret_cast<_Float16*>(take(size_t(T) * pf_np(n) * 2));
    w.xlo = reinterpret_cast<_Float16*>(take(size_t(T) * pf_np(n) * 2));
    w.h16 = reinterpret_cast<_Float16*>(take(size_t(S) * ((ff + 255) & ~255) * 2));
    // (fp32 when ff > 1024: the down GEMM's chunks are added up in it)
    w.yd = own_yd ? reinterpret_cast<_Float16*>(take(size_t(S) * n * (ff > 1024 ? 4 : 2))) : nullptr;
    w.bytes = size_t(p - static_cast<uint8_t*>(base));
    return w;
}

size_t pf_workspace_bytes(int T, int K, int n, int ff, int E, bool shared, bool own_yd) {
    return pf_carve(nullptr, T, K, n, ff, E, shared, own_yd).bytes + 256;
}

int quantize_pairs(const float* x, int rows, int n, int np, int blk, _Float16* xhi, _Float16* xlo, hipStream_t stream);

int pf_check(int T, int K, int n, int ff, int E) {
    if (T < 1 || K < 1 || K > 32 || E < 1 || E > 4096 || K > E) return set_error(kErrShape, "prefill: T=%d K=%d E=%d", T, K, E);
    // n and ff multiples of 128 (moe_q2.cu:516-517); gate/up: slices of 128 ff rows; down: the tile's
    // h (ff rounded up to 256) in LDS in chunks of at most 1024
    if (n % 128 || n < 128 || n > 65536 || ff % 128 || ff < 128 || ff > 4096)
        return set_error(kErrShape, "prefill: n=%d ff=%d (n and ff multiples of 128; ff at most 4096)", n, ff);
    return kOk;
}

template <bool SMALL>
static int pf_gemm_attr() {
    static bool done = false;   // per process; the attribute is a property of the kernel
    if (!done) {
        FRT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm<SMALL>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, GuShape<SMALL>::smem));
        done = true;
    }
    return kOk;
}

template <int NQ, bool TAIL, typename OutT, bool SMALL>
static int pf_down_attr(size_t lds) {
    static bool done = false;
    if (!done) {
        FRT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_down<NQ, TAIL, OutT, SMALL>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
        done = true;
    }
    return kOk;
}

// The two grouped GEMMs: gate/up (k_pf_gemm) on the exact x pairs, SwiGLU and Q8_0 of h in the
// epilogue; down (k_pf_down) on h -> yd per slot as OutT.
template <typename OutT>
static int pf_expert_gemms(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff,
                           int blk, const PfWs& w, int mt, OutT* ydf, hipStream_t stream) {
    if (int rc = pf_gemm_attr<false>()) return rc;
    if (int rc = pf_gemm_attr<true>()) return rc;
    // tiles of 2-4 token columns, then those of one (the tile list is ordered longest first)
    const int mt8 = (mt + 7) / 8 * 8;
    launch_timed("pf_gateup", k_pf_gemm<false>, dim3(ff / GuShape<false>::ff_rows * mt8), dim3(GuShape<false>::threads),
                 GuShape<false>::smem, stream, arena, stride, E, shared_blob, n, pf_np(n), blk, ff, (const _Float16*)w.xhi,
                 (const _Float16*)w.xlo, (const int32_t*)w.tok_of, (const int32_t*)w.bounds, (const int2*)w.tiles,
                 (const int32_t*)w.n_tiles, w.h16);
    launch_timed("pf_gateup1", k_pf_gemm<true>, dim3(ff / GuShape<true>::ff_rows * mt8), dim3(GuShape<true>::threads),
                 GuShape<true>::smem, stream, arena, stride, E, shared_blob, n, pf_np(n), blk, ff, (const _Float16*)w.xhi,
                 (const _Float16*)w.xlo, (const int32_t*)w.tok_of, (const int32_t*)w.bounds, (const int2*)w.tiles,
                 (const int32_t*)w.n_tiles, w.h16);
    timing_mark(stream, "pf_gateup");
    const int ffp = (ff + 255) / 256 * 256;   // h row length
    // ff up to 1024: one pass over the whole h row; beyond, chunks of 1024 added up in fp32 yd
    if (ffp > 1024 && !std::is_same<OutT, float>::value)
        return set_error(kErrShape, "prefill: ff=%d above 1024 needs fp32 per-slot outputs", ff);
    for (int k0 = 0; k0 < ffp; k0 += 1024) {
        const int nq = (ffp - k0 < 1024 ? ffp - k0 : 1024) / 256;   // stretches of this chunk
        const size_t down_lds = size_t(kTN) * nq * 256 * 2;         // the tile's activations (SMALL: a quarter)
        const bool tail = ((n + 255) / 256) * nq % 4 != 0;
        const int acc = k0 > 0 ? 1 : 0;
#define FRT_PF_DOWN(NQV, TL)                                                                                 \
    if (nq == NQV && tail == TL) {                                                                           \
        if (int rc = pf_down_attr<NQV, TL, OutT, false>(down_lds)) return rc;                                \
        if (int rc = pf_down_attr<NQV, TL, OutT, true>(down_lds / 4)) return rc;                             \
        launch_timed("pf_down", k_pf_down<NQV, TL, OutT, false>, dim3(1, mt), dim3(256), down_lds, stream, arena, \
                     stride, E, shared_blob, n, ff, (const _Float16*)w.h16, (const int32_t*)w.bounds,            \
                     (const int2*)w.tiles, (const int32_t*)w.n_tiles, ydf, (const int32_t*)w.slot_of, k0, ffp, acc); \
        launch_timed("pf_down1", k_pf_down<NQV, TL, OutT, true>, dim3(1, mt), dim3(256), down_lds / 4, stream, arena, \
                     stride, E, shared_blob, n, ff, (const _Float16*)w.h16, (const int32_t*)w.bounds,            \
                     (const int2*)w.tiles, (const int32_t*)w.n_tiles, ydf, (const int32_t*)w.slot_of, k0, ffp, acc); \
    }
        FRT_PF_DOWN(1, false) FRT_PF_DOWN(1, true) FRT_PF_DOWN(2, false) FRT_PF_DOWN(2, true)
        FRT_PF_DOWN(3, false) FRT_PF_DOWN(3, true) FRT_PF_DOWN(4, false) FRT_PF_DOWN(4, true)
#undef FRT_PF_DOWN
    }
    return kOk;
}

// The grouped expert products for routed ids (+ optionally the shared expert as group E).
// yd_kind: 0 float, 1 bf16 (moe_q2::run's yd_bf16), 2 fp16 (a whole layer's, combined here)
static int pf_experts(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff,
                      const float* x, const int32_t* ids, int T, int K, void* yd, int yd_kind, int blk, const PfWs& w,
                      hipStream_t stream) {
    const bool shared = shared_blob != nullptr;
    const int S = T * K + (shared ? T : 0);
    const int G = E + (shared ? 1 : 0);
    const int nchunk = (T * K + kChunk - 1) / kChunk;
    int id_bits = 1;
    while ((1 << id_bits) < E) ++id_bits;
    if (int rc = quantize_pairs(x, T, n, pf_np(n), blk, w.xhi, w.xlo, stream)) return rc;
    timing_mark(stream, "pf_quant_x");
    launch_timed("pf_hist", k_pf_hist, dim3(nchunk), dim3(256), size_t(E) * 4, stream, ids, T * K, E, w.cnt);
    launch_timed("pf_colscan", k_pf_colscan, dim3((E + 3) / 4), dim3(256), 0, stream, w.cnt, nchunk, E, w.bounds);
    launch_timed("pf_scan", k_pf_scan, dim3(1), dim3(1024), 0, stream, E, T, shared ? 1 : 0, w.bounds, w.tiles,
                 w.n_tiles);
    launch_timed("pf_place", k_pf_place, dim3(nchunk + (shared ? (T + 63) / 64 : 0)), dim3(64), size_t(E) * 4, stream,
                 ids, T * K, K, E, id_bits, (const int32_t*)w.cnt, (const int32_t*)w.bounds, w.tok_of, w.slot_of,
                 shared ? T : 0);
    timing_mark(stream, "pf_dispatch");
    const int mt = pf_max_tiles(S, G);
    int rc = kOk;
    if (yd_kind == 1) rc = pf_expert_gemms(arena, stride, E, shared_blob, n, ff, blk, w, mt, static_cast<__hip_bfloat16*>(yd), stream);
    else if (yd_kind == 2) rc = pf_expert_gemms(arena, stride, E, shared_blob, n, ff, blk, w, mt, static_cast<_Float16*>(yd), stream);
    else rc = pf_expert_gemms(arena, stride, E, shared_blob, n, ff, blk, w, mt, static_cast<float*>(yd), stream);
    if (rc) return rc;
    timing_mark(stream, "pf_down");
    FRT_LAUNCHED("prefill experts");
    return kOk;
}

// moe_q2::run (kernels/cuda/moe_q2.h:20-30): yd [T*K][n] per slot
int pf_run(const uint8_t* experts, size_t stride, int E, int n, int ff, const float* x, const int32_t* ids, int T, int K,
           void* yd, void* ws, size_t ws_bytes, hipStream_t stream, int block64, int yd_bf16) {
    if (int rc = pf_check(T, K, n, ff, E)) return rc;
    if (!experts || !x || !ids || !yd || !ws) return set_error(kErrNull, "moe_q2::run: null pointer");
    const PfWs w = pf_carve(ws, T, K, n, ff, E, false, false);
    if (w.bytes > ws_bytes) return set_error(kErrWorkspace, "moe_q2::run: workspace %zu < %zu", ws_bytes, w.bytes);
    // block64: x and h quantized in Q8_0 blocks of 64 values rather than 32 (moe_q2.cu's AB = 64)
    return pf_experts(experts, stride, E, nullptr, n, ff, x, ids, T, K, yd, yd_bf16 ? 1 : 0, block64 ? 64 : 32, w, stream);
}

// The whole prefill layer after routing: ids/wts [T][K], gate [T] -> out [T][n] (+ resid)
int pf_moe(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff, const float* x,
           const int32_t* ids, const float* wts, const float* gate, int T, int K, const float* resid, float* out,
           void* ws, size_t ws_bytes, hipStream_t stream) {
    if (int rc = pf_check(T, K, n, ff, E)) return rc;
    const PfWs w = pf_carve(ws, T, K, n, ff, E, true, true);
    if (w.bytes > ws_bytes) return set_error(kErrWorkspace, "prefill: workspace %zu < %zu", ws_bytes, w.bytes);
    if (ff > 1024) {   // fp32 per-slot outputs
        if (int rc = pf_experts(arena, stride, E, shared_blob, n, ff, x, ids, T, K, w.yd, 0, 32, w, stream)) return rc;
        launch_timed("pf_combine", k_pf_combine<float>, dim3((n + 1023) / 1024, T), dim3(256), 0, stream,
                     (const float*)w.yd, ids, wts, gate, T, K, n, 1, resid, out);
        timing_mark(stream, "pf_combine");
        FRT_LAUNCHED("prefill combine");
        return kOk;
    }
    if (int rc = pf_experts(arena, stride, E, shared_blob, n, ff, x, ids, T, K, w.yd, 2, 32, w, stream)) return rc;
    launch_timed("pf_combine", k_pf_combine<_Float16>, dim3((n + 1023) / 1024, T), dim3(256), 0, stream,
                 (const _Float16*)w.yd, ids, wts, gate, T, K, n, 1, resid, out);
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
    k_pf_colscan<<<(E + 3) / 4, 256, 0, stream>>>(cnt, nchunk, E, bounds);
    k_pf_scan<<<1, 1024, 0, stream>>>(E, T, 0, bounds, tiles, n_tiles);
    k_pf_place<<<nchunk, 64, size_t(E) * 4, stream>>>(ids, T * K, K, E, id_bits, cnt, bounds, tok_of, slot_of, 0);
    FRT_LAUNCHED("dispatch");
    return kOk;
}
size_t pf_dispatch_ws_bytes(int T, int K, int E) {
    const int nchunk = (T * K + kChunk - 1) / kChunk;
    return up256(size_t(nchunk) * E * 4) + up256(size_t(pf_max_tiles(T * K, E)) * 8) + 256;
}

}  // namespace frt
