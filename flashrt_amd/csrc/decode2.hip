// Single-token MoE layers (T = 1 decode) as ONE persistent launch, with the work of each layer split
// by XCD so that most joins between workgroups stay inside one XCD's L2.
//
// The same layer as decode1.hip (moe_block_fast, arch/qwen4exp/moe_fast.cu:1015-1108; the phase A /
// phase B split of quant/q2_0/moe_cpu.cpp:36-114), on a grid of one 512-thread workgroup per CU,
// all resident together. Workgroup b runs on XCD x = b mod 8 as workgroup j = b / 8 of the XCD's NL.
// Per layer:
//   1. router: workgroup b computes router rows b, b + G, ... (one wave per row, the canonical order
//      of route.hip) and publishes them (cross-XCD words); workgroup j of every XCD then relays logits
//      j lc .. j lc + lc - 1 into its XCD's L2, where every workgroup of the XCD reads all E + 1.
//   2. every workgroup routes the token itself (route1_wave). The K + 1 entries (routed in ascending
//      id, the shared expert last) are split over the XCDs: entry u < 8 floor((K+1)/8) is owned by
//      XCD u mod 8 (all ff rows), each remaining entry is split by ff rows (32-row blocks, about ff/8
//      per XCD). An XCD's (entry, ff row) pairs are split over its workgroups: gate and up rows,
//      SwiGLU, the h value published in the XCD's L2.
//   3. every workgroup of the XCD reads the XCD's h values, quantizes them (Q8_0 per 32, as the CPU
//      path), and computes its n / NL down rows over the XCD's part of ff for every entry of the
//      XCD: the owned entries' whole rows, the split entries' XCD slice. It weighs them by the
//      routing weights (sigmoid(gate) for the shared expert) and publishes each row's XCD partial.
//   4. workgroup j of every XCD gathers the 8 XCD partials of rows j n/NL .. (j+1) n/NL - 1, sums them
//      (((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7))), adds the layer input (a stack) or the residual, and
//      publishes the rows in its XCD's L2: the next layer's input.
// Two joins per layer cross XCDs (the logits, the partials), each read by one workgroup per XCD and
// word; the rest are read from the XCD's own L2. The float order of the down sums and of the
// combine differs from decode1.hip's (the XCD partials are summed last); the outputs are within the
// layer bar of the CPU path, not bit-equal to decode1.hip's.
// Joins, epochs and the bounded waits are those of persist.hpp (every wait bounded; a call out of
// time sets the error words and finishes).
#include <hip/hip_runtime.h>

// threadIdx.x read through an empty volatile asm (see decode1.hip): values derived from it are
// computed where they are used rather than hoisted out of the layer loop.
struct FrtOpaqueTid2 {
    __device__ unsigned get_x() const {
        unsigned t = __builtin_amdgcn_workitem_id_x();
        asm volatile("" : "+v"(t));
        return t;
    }
    __declspec(property(get = get_x)) unsigned x;
};
#define threadIdx (FrtOpaqueTid2{})
#include "decode_parts.hpp"
#include "persist.hpp"

#include "../../include/flashrt_moe.h"

#include <map>
#include <mutex>
#include <set>
#include <utility>

namespace frt {

constexpr int kLgStride2 = 4;   // words between two cross-XCD logits (the same as decode1.hip)

namespace {

constexpr int kNT2 = kNTP;
constexpr int kNW2 = kNT2 / 64;
constexpr int kMaxRW = 128;     // down rows per workgroup (n / NL)
// Roles of the waves around each join. A wave's wait for a load also waits for every store it
// issued before that load (one counter for both, completed in order), and a store that other XCDs
// read is acknowledged only from beyond the XCD's L2: so no wave polls a join soon after it published
// a word, and no wave polls while its router-row loads for the next layer are in flight.
//   logits: waves 0-2 publish them (router rows); wave 3 relays; waves 4-7 read the XCD's copy;
//   h: every wave computes gate/up into LDS; wave 7 publishes the workgroup's h values; waves 0-6
//      read the XCD's;
//   partials: waves 0-1 publish; waves 2-7 gather the rows' 8 partials; waves 0-1 then publish the
//   next layer's input rows; waves 2-7 read them at the next layer's start.
constexpr int kRelayT0 = 0;     // the logit relay's threads (wave 3)
constexpr int kPollT0 = 0;      // threads from here read the relayed logits (waves 4-7)
constexpr int kHPubW = 7;       // the wave publishing the workgroup's h values
constexpr int kDT = kNTP;       // the down rows' threads
constexpr int kHPollT0 = 0;     // threads from here read the XCD's h values (waves 0-6)
constexpr int kMaxPx = 4096;    // h values per XCD, at most
constexpr int kXPollT0 = 0;     // threads from here gather the partials and read the next input

struct Dec2Args {
    Dec1Layer lay[kMaxStack];
    int n_layer;           // 1: one layer (resid optional); more: a stack, x_{l+1} = x_l + moe_l(x_l)
    const float* x;        // [n] the (first) layer's input
    size_t stride;
    const float* resid;    // [n] or null (one layer)
    float* out;            // [n] the (last) layer's output
    int32_t* ids;          // [n_layer][K] rank order, or null
    float* wts;            // [n_layer][K], or null
    uint32_t* counts;      // [E] or null (one layer)
    Dec1Sync* sync;
    uint64_t* lg;          // [E + 1] cross-XCD logits, kLgStride2 words apart (the shared gate last)
    uint64_t* lgl;         // [8][kD2LglWords] the logits relayed into each XCD
    uint64_t* hl;          // [8][kD2HlWords] each XCD's h values, in its pair order
    uint64_t* xp;          // [8][kD2XWords] each XCD's weighted down partials per output row
    uint64_t* xl;          // [8][kD2XWords] the next layer's input, relayed into each XCD
    const float* next_w;   // the next call's router [E][n] (cache warming) or null
    uint64_t ticks;        // bound of the call's waits, in ticks of the 100 MHz constant clock
    uint32_t* host_err;
    uint64_t* stamps;      // measurement only (null: none): [layer][phase][workgroup] constant-clock ticks
    int route8;            // the single-token routing by all 8 waves (route_8waves) rather than one
    int E, K, ff, nbf, norm;
};

typedef const __attribute__((address_space(4))) Dec2Args KArgs2;
typedef const __attribute__((address_space(4))) Dec1Layer KLayer2;

// The XCD's part of the layer's experts: owned entries x, x + 8, ... (all ff rows) and the split
// entries' 32-row blocks hb0 .. hb1 - 1. Pair p of the XCD (an ff row of an entry, gate and up):
// the owned entries' rows first, then the split entries' slices.
struct XcdPart {
    int nown, nsplit, hb0, hb1, rs, px;
    __device__ XcdPart(int U, int ff, int xcd) {
        nown = U >> 3;
        nsplit = U & 7;
        const int nbh = ff / 32;
        hb0 = (xcd * nbh) >> 3;
        hb1 = ((xcd + 1) * nbh) >> 3;
        rs = 32 * (hb1 - hb0);
        px = nown * ff + nsplit * rs;
    }
    // entry and ff row of pair p
    __device__ void pair(int p, int ff, int xcd, int& u, int& row) const {
        if (p < nown * ff) {
            u = xcd + 8 * (p / ff);
            row = p % ff;
        } else {
            const int q = p - nown * ff;
            u = 8 * nown + q / rs;
            row = 32 * hb0 + q % rs;
        }
    }
};

constexpr int kD2Phases = 12;
// (kept in LDS and written out at the end: a store in the layer would delay the wave's next wait)
#define FRT_D2_STAMP(ph)                                                                                    \
    do {                                                                                                    \
        if (a.stamps && threadIdx.x == 0) s_stamp[l][ph] = wall_clock64();                                 \
    } while (0)

template <int NB, int V, bool STACK>
__global__ void __launch_bounds__(kNT2) k_dec2(Dec2Args a_byval) {
    (void)a_byval;
    const KArgs2& a = *(const KArgs2*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int n = 64 * NB, L = NB;   // the router's 64 chains are L = n / 64 long
    // dynamic: h_f [px] float | sh_q [px] int8 | sh_d [px / 32] float | sy [nseg][RW] float
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float xs[64 * (L + 1)];   // x by chain, each chain padded by one float
    __shared__ __align__(16) int8_t xq[n];
    __shared__ float xd[n / kQ8];
    __shared__ __align__(16) float s_lg[64 * V + 4];
    __shared__ WinLds R;
    __shared__ Route8Lds s_q8;
    __shared__ float s_part[8][kMaxRW];
    __shared__ uint64_t s_stamp[kMaxStack][kD2Phases];

    const int b = blockIdx.x, G = gridDim.x;
    const int xcd = b & 7, j = b >> 3, NL = G >> 3;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = a.E, K = a.K, ff = a.ff, U = K + 1, NBF = a.nbf;
    const int RW = n / NL, r0 = j * RW;   // this workgroup's down rows, and the rows it relays
    const XcdPart X(U, ff, xcd);
    const int p0 = (j * X.px) / NL, p1 = ((j + 1) * X.px) / NL;   // this workgroup's pairs
    float* h_f = reinterpret_cast<float*>(smem);
    int8_t* sh_q = reinterpret_cast<int8_t*>(smem + size_t(X.px) * 4);
    float* sh_d = reinterpret_cast<float*>(smem + size_t(X.px) * 5);
    float* sy = sh_d + X.px / 32;
    uint64_t* LGL = a.lgl + size_t(xcd) * kD2LglWords;
    uint64_t* HL = a.hl + size_t(xcd) * kD2HlWords;
    uint64_t* XL = a.xl + size_t(xcd) * kD2XWords;
    const uint64_t deadline = wall_clock64() + a.ticks;
    __shared__ uint32_t s_ep[kNW2];
    {
        uint32_t c = tid < G ? __hip_atomic_load(&a.sync->epoch[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        if (G > kNT2)
            for (int i = tid + kNT2; i < G; i += kNT2)
                c = max(c, __hip_atomic_load(&a.sync->epoch[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        for (int o = 32; o > 0; o >>= 1) c = max(c, uint32_t(__shfl_xor(int(c), o, 64)));
        if (lane == 0) s_ep[wave] = c;
    }

    // ---- router rows (slot s = b + G w for wave w; slot E is the shared gate row). The wave index is
    // taken as a scalar, so that the branches on it are uniform and their loads need no wait where
    // they join.
    const int s0 = b + __builtin_amdgcn_readfirstlane(tid >> 6) * G;
    const bool rs = s0 <= E;
    float wr[L];
    float bias_v = 0.0f;
    // (the next layer's rows are loaded right after this layer's router dot, so that they land
    // during the rest of the layer; the waves holding router rows then poll no word of the layer
    // before those loads are in: a poll waits for every load its wave issued before it)
    auto load_router = [&](const Dec1Layer& LY) {
        if (rs) {
            const float* wrow = s0 < E ? LY.W + size_t(s0) * n : LY.gate_w;
            const float4* w4 = reinterpret_cast<const float4*>(wrow + lane * L);
#pragma unroll
            for (int i = 0; i < L / 4; ++i) {
                const float4 v = w4[i];
                wr[4 * i] = v.x;
                wr[4 * i + 1] = v.y;
                wr[4 * i + 2] = v.z;
                wr[4 * i + 3] = v.w;
            }
        }
        const float* bp = LY.bias ? LY.bias + min(s0, E - 1) : LY.gate_w;   // (always a valid address)
        const float bv = *bp;
        bias_v = LY.bias ? bv : 0.0f;
        // the loads are issued here, not sunk to their use in the next layer (this orders them
        // before every later memory access; nothing waits for them here)
        asm volatile("" ::: "memory");
    };
    {
        Dec1Layer l0;
        l0.W = a.lay[0].W;
        l0.gate_w = a.lay[0].gate_w;
        l0.bias = a.lay[0].bias;
        load_router(l0);
    }
    constexpr int XV = (n / 4 + kNT2 - 1) / kNT2;
    float4 xv[XV];
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
#pragma unroll
    for (int k = 0; k < XV; ++k) xv[k] = x4[min(tid + k * kNT2, n / 4 - 1)];
    const float res = (!STACK && a.resid && tid < RW) ? a.resid[r0 + tid] : 0.0f;
#pragma unroll
    for (int k = 0; k < XV; ++k) {
        const int idx = tid + k * kNT2;
        if (idx < n / 4) {
            const int e = 4 * idx;   // L % 4 == 0: a float4 stays within one chain
            float* d = xs + (e / L) * (L + 1) + e % L;
            d[0] = xv[k].x;
            d[1] = xv[k].y;
            d[2] = xv[k].z;
            d[3] = xv[k].w;
        }
    }
    __syncthreads();
    uint32_t ep = s_ep[0];
#pragma unroll
    for (int w = 1; w < kNW2; ++w) ep = max(ep, s_ep[w]);
    ep += 1u;
    const uint64_t err_val = (uint64_t(kErrMagic) << 32) | ep;
    uint64_t* const errw = &a.sync->err;
    const int n_layer = STACK ? a.n_layer : 1;
    for (int l = 0; l < n_layer; ++l) {
    const KLayer2& LY = a.lay[l];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;   // per layer (see FrtOpaqueTid2)
    const uint32_t tag = sync_tag(ep * uint32_t(kMaxStack) + uint32_t(l));
    if (l > 0) {   // x_l from the previous layer's relay in this XCD
        __syncthreads();   // the previous layer has read xs
        if (tid >= kXPollT0)
            wait_words_at<(kD2XWords + kNT2 - kXPollT0 - 1) / (kNT2 - kXPollT0), kNT2 - kXPollT0>(
                [&](int i) { return XL + i; }, n, tag, deadline, errw, err_val, a.host_err,
                [&](int i, uint32_t p) { xs[(i / L) * (L + 1) + i % L] = __uint_as_float(p); }, kXPollT0);
        __syncthreads();
    }
    FRT_D2_STAMP(0);
    const float r = a.norm ? rms_scale_wave<L>(xs + lane * (L + 1), n) : 1.0f;
    FRT_D2_STAMP(9);
    auto router_dot = [&](int s, const float (&w)[L], float bv) {
        const float* xc = xs + lane * (L + 1);
        float acc = 0.0f;
        if (a.norm) {
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const float u = xc[i] * r;
                acc = fmaf(w[i], u, acc);
            }
        } else {
#pragma unroll
            for (int i = 0; i < L; ++i) acc = fmaf(w[i], xc[i], acc);
        }
        acc = wave_sum_tree(acc);
        if (s < E && LY.bias) acc = acc + bv;
        if (lane == 0) pub(a.lg + size_t(s) * kLgStride2, tag, __float_as_uint(acc));
    };
    if (rs) router_dot(s0, wr, bias_v);
    FRT_D2_STAMP(10);
    // the next layer's router rows (a stack), or the next call's into this XCD's L2 (warming; without
    // one, this layer's rows again), by one load statement: one definition of wr in the loop, so that
    // no register copy waits for the loads here
    {
        const bool more = l + 1 < n_layer;
        Dec1Layer nl;
        nl.W = more ? a.lay[l + 1].W : (a.next_w ? a.next_w : LY.W);
        nl.gate_w = more ? a.lay[l + 1].gate_w : LY.gate_w;
        nl.bias = more ? a.lay[l + 1].bias : nullptr;
        load_router(nl);
    }
    for (int s = s0 + kNW2 * G; s <= E; s += kNW2 * G) {   // only with fewer than (E + 1) / 8 workgroups
        float w2[L];
        const float* wrow = s < E ? LY.W + size_t(s) * n : LY.gate_w;
#pragma unroll
        for (int i = 0; i < L; ++i) w2[i] = wrow[lane * L + i];
        router_dot(s, w2, LY.bias && s < E ? LY.bias[s] : 0.0f);
    }
    // Q8_0 of the experts' input (u = x r with the norm) by the last two waves: a lane pair per 32-block
    if (wave >= kNW2 - 2) {
        const int h = lane & 1;
        for (int b0 = (wave - (kNW2 - 2)) * 32; b0 < n / kQ8; b0 += 64) {
            const int blk = min(b0 + (lane >> 1), n / kQ8 - 1);
            float v[16];
            float am = 0.0f;
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const int k = blk * kQ8 + 16 * h + jj;
                v[jj] = xs[(k / L) * (L + 1) + k % L];
                if (a.norm) v[jj] = v[jj] * r;
                am = fmaxf(am, fabsf(v[jj]));
            }
            am = fmaxf(am, FRT_DPP(am, kDppXor1));
            const float d = q8_scale(am);
            const float id = q8_inv(d);
            uint32_t wq[4];
#pragma unroll
            for (int w = 0; w < 4; ++w)
                wq[w] = uint32_t(q8_code(v[4 * w], id) & 0xff) | (uint32_t(q8_code(v[4 * w + 1], id) & 0xff) << 8) |
                        (uint32_t(q8_code(v[4 * w + 2], id) & 0xff) << 16) | (uint32_t(q8_code(v[4 * w + 3], id) & 0xff) << 24);
            if (b0 + (lane >> 1) < n / kQ8) {
                uint32_t* dst = reinterpret_cast<uint32_t*>(xq + blk * kQ8 + 16 * h);
#pragma unroll
                for (int w = 0; w < 4; ++w) dst[w] = wq[w];
                if (h == 0) xd[blk] = f16_round(d);
            }
        }
    }

    FRT_D2_STAMP(1);
    // ---- the logits: relay this workgroup's share into the XCD, then read all from the XCD's L2
    {
        const int lc = (E + 1 + NL - 1) / NL;
        for (int rt = tid - kRelayT0, i = j * lc + rt; rt >= 0 && rt < lc && tid < kRelayT0 + 64 && i <= E;
             rt += 64, i += 64) {
            const uint64_t* src = a.lg + size_t(i) * kLgStride2;
            uint64_t v = peek(src);
            while (uint32_t(v >> 32) != tag) {
                __builtin_amdgcn_s_sleep(2);
                if (wall_clock64() > deadline) {
                    __hip_atomic_store(errw, err_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (a.host_err) __hip_atomic_store(a.host_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    v = (uint64_t(tag) << 32) | uint32_t(v);
                    break;
                }
                v = peek(src);
            }
            pub_local(LGL + i, tag, uint32_t(v));
        }
    }
    FRT_D2_STAMP(2);
    if (tid >= kPollT0)
        wait_words_at<(1024 + 1 + kNT2 - kPollT0 - 1) / (kNT2 - kPollT0), kNT2 - kPollT0>(
            [&](int i) { return LGL + i; }, E + 1, tag, deadline, errw, err_val, a.host_err,
            [&](int i, uint32_t p) { s_lg[i] = __uint_as_float(p); }, kPollT0);
    FRT_D2_STAMP(3);
    if (E <= 512 && kPollT0 == 0 && a.route8) {   // the 8 waves route together (each may start on its own logits)
        route_8waves(s_lg, E, K, LY.arena, a.stride, LY.shared, R, s_q8);
    } else {
    __syncthreads();
    if (wave == 0) {
        float v[V];
        if (E == 64 * V) {
#pragma unroll
            for (int i = 0; i < V / 4; ++i) {
                const float4 q = reinterpret_cast<const float4*>(s_lg + V * lane)[i];
                v[4 * i] = q.x;
                v[4 * i + 1] = q.y;
                v[4 * i + 2] = q.z;
                v[4 * i + 3] = q.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) v[i] = s_lg[min(V * lane + i, E - 1)];   // past E: masked by the keys
        }
        route1_wave<V, true>(v, E, K, s_lg[E], LY.arena, a.stride, LY.shared, R);
    }
    }
    FRT_D2_STAMP(11);
    __syncthreads();
    if (R.many) {   // more than 64 candidates (heavily tied logits): four waves select, as window_entries
        float mx;
        topk_group4<V>(s_lg, E, K, wave & 3, wave < 4, R.tk[0], mx);
        if (wave == 0) {
            const float sel_l = lane < K ? R.tk[0].sel_v[lane] : 0.0f;
            const int sel_id = lane < K ? R.tk[0].sel_id[lane] : 0x7fffffff;
            int u = 0;
            for (int jj = 0; jj < K; ++jj) u += int(__builtin_amdgcn_readlane(sel_id, jj) < sel_id);
            if (lane < K) {
                R.ids[0][lane] = sel_id;
                R.w[0][lane] = sel_l;
                DecEntry& d = R.ent[u];
                d.blob = LY.arena + size_t(sel_id) * a.stride;
                d.ntok = 1;
                d.base = u;
                d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
                d.slot[0] = lane;
                d.slot[1] = d.slot[2] = d.slot[3] = -1;
                d.w[0] = sel_l;
                d.w[1] = d.w[2] = d.w[3] = 0.0f;
            } else if (lane == K) {
                DecEntry& d = R.ent[K];
                d.blob = LY.shared;
                d.ntok = 1;
                d.base = K;
                d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
                d.slot[0] = d.slot[1] = d.slot[2] = d.slot[3] = -1;
                d.w[0] = s_lg[E];
                d.w[1] = d.w[2] = d.w[3] = 0.0f;
            }
        }
        __syncthreads();
    }

    // ---- gate/up of this workgroup's pairs p0 .. p1 - 1, RPW rows per wave pass, 2 passes per batch
    constexpr int RPW = gu_rpw<NB>();
    constexpr int SLOTS = kNW2 * RPW;
    constexpr int PB = 2;
    __shared__ __align__(16) float seqbuf[kNW2][PB * 128];   // per wave: the block terms of seq_row_sums
    const int rsub = lane / NB, bk = lane % NB;
    const bool live = rsub < RPW;
    const int bl = live ? bk : 0;
    const int slot = wave * RPW + rsub;
    const size_t mb = mat_bytes(ff, n);
    uint4 cg[PB], cu[PB];
    uint32_t sg[PB], su[PB];
    uint32_t okm = 0;
    auto gu_load = [&](int pb) {
        okm = 0;
#pragma unroll
        for (int k = 0; k < PB; ++k) {
            const int p = pb + k * SLOTS + slot;
            const bool ok = live && p < p1;
            if (ok) okm |= 1u << k;
            int u, row;
            X.pair(ok ? p : p0, ff, xcd, u, row);
            const uint8_t* blob = R.ent[u].blob;
            const uint8_t* gcodes = blob;
            const uint16_t* gscal = reinterpret_cast<const uint16_t*>(blob + size_t(ff) * NB * 16);
            const uint8_t* ucodes = blob + mb;
            const uint16_t* uscal = reinterpret_cast<const uint16_t*>(blob + mb + size_t(ff) * NB * 16);
            cg[k] = gld_u4_nt(gcodes + (size_t(row) * NB + bl) * 16);
            cu[k] = gld_u4_nt(ucodes + (size_t(row) * NB + bl) * 16);
            sg[k] = gld<uint16_t>(gscal + size_t(row) * NB + bl);
            su[k] = gld<uint16_t>(uscal + size_t(row) * NB + bl);
        }
    };
    auto gu_compute = [&](int pb) {
        int xa[16];
        const int4* xp = reinterpret_cast<const int4*>(xq + bl * kBlock);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int4 v = xp[k];
            xa[4 * k] = v.x;
            xa[4 * k + 1] = v.y;
            xa[4 * k + 2] = v.z;
            xa[4 * k + 3] = v.w;
        }
        const float xd0 = xd[2 * bl], xd1 = xd[2 * bl + 1];
        int xs0 = 0, xs1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) xs0 = dot4(xa[i], 0x01010101, xs0);
#pragma unroll
        for (int i = 8; i < 16; ++i) xs1 = dot4(xa[i], 0x01010101, xs1);
        float tg[PB], tu[PB];
#pragma unroll
        for (int k = 0; k < PB; ++k) {
            const uint32_t wg[4] = {cg[k].x, cg[k].y, cg[k].z, cg[k].w};
            const uint32_t wu[4] = {cu[k].x, cu[k].y, cu[k].z, cu[k].w};
            const bool okp = (okm >> k) & 1u;
            const float dg = okp ? h2f(uint16_t(sg[k])) : 0.0f, du = okp ? h2f(uint16_t(su[k])) : 0.0f;
            int g0 = 0, g1 = 0, u0 = 0, u1 = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                g0 = dot4(int(wg[w] & 0x03030303u), xa[w], g0);
                g0 = dot4(int((wg[w] >> 2) & 0x03030303u), xa[4 + w], g0);
                g1 = dot4(int((wg[w] >> 4) & 0x03030303u), xa[8 + w], g1);
                g1 = dot4(int((wg[w] >> 6) & 0x03030303u), xa[12 + w], g1);
                u0 = dot4(int(wu[w] & 0x03030303u), xa[w], u0);
                u0 = dot4(int((wu[w] >> 2) & 0x03030303u), xa[4 + w], u0);
                u1 = dot4(int((wu[w] >> 4) & 0x03030303u), xa[8 + w], u1);
                u1 = dot4(int((wu[w] >> 6) & 0x03030303u), xa[12 + w], u1);
            }
            const float fg = float(g0 - xs0) * xd0 + float(g1 - xs1) * xd1;
            const float fu = float(u0 - xs0) * xd0 + float(u1 - xs1) * xd1;
            tg[k] = fg * dg;
            tu[k] = fu * du;
        }
        // the rows' sums in the CPU path's order: lane 2 RPW k + r holds pair pb + k SLOTS + wave RPW + r
        const float2 gu = seq_row_sums<NB, RPW, PB>(tg, tu, seqbuf[wave], lane);
        const int k = lane / (2 * RPW), r = lane % (2 * RPW);
        const int p = pb + k * SLOTS + wave * RPW + r;
        if (r < RPW && k < PB && p < p1) h_f[p] = gu.x / (1.0f + expf(-gu.x)) * gu.y;   // published below by one wave
    };

    // ---- down: this workgroup's rows r0 .. r0 + RW - 1 over the XCD's part of ff. Owned entries: one
    // lane per (row, 64-block), NBF lanes per row; split entries: one lane per (row, entry) over the
    // XCD's blocks (NCH 64-blocks at most).
    constexpr int DOB = 2;   // owned down loads per thread issued ahead
    constexpr int NCH = 2;   // 64-blocks per split row and XCD, at most (ff <= 1024)
    const int nown_items = X.nown * RW * NBF;
    const int nsplit_items = X.nsplit * RW;
    const int cb0 = X.hb0 >> 1, cb1 = (X.hb1 + 1) >> 1;   // the split entries' 64-blocks in this XCD
    const size_t dbase = 2 * mb;
    uint4 dco[DOB];
    uint32_t dso[DOB];
    uint4 dcs[NCH];
    uint32_t dss[NCH];
    auto own_load = [&](int it0) {
#pragma unroll
        for (int k = 0; k < DOB; ++k) {
            const int it = min(it0 + tid + k * kDT, nown_items - 1);
            const int m = it / (RW * NBF), rem = it % (RW * NBF);
            const int rr = rem / NBF, c = rem % NBF;
            const uint8_t* db = R.ent[xcd + 8 * m].blob + dbase;
            dco[k] = gld_u4_nt(db + (size_t(r0 + rr) * NBF + c) * 16);
            dso[k] = gld<uint16_t>(db + size_t(n) * NBF * 16 + (size_t(r0 + rr) * NBF + c) * 2);
        }
    };
    auto split_load = [&](int it) {   // item it < nsplit_items
        const int s = it / RW, rr = it % RW;
        const uint8_t* db = R.ent[8 * X.nown + s].blob + dbase;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int cc = min(cb0 + c, cb1 - 1);
            dcs[c] = gld_u4_nt(db + (size_t(r0 + rr) * NBF + cc) * 16);
            dss[c] = gld<uint16_t>(db + size_t(n) * NBF * 16 + (size_t(r0 + rr) * NBF + cc) * 2);
        }
    };
    // the 64-block c of a down row against h codes hq (the block's 64 codes, or its halves' bases
    // h0 / h1 with their scales; a half outside the XCD counts 0)
    auto chunk_dot = [&](const uint4& wdv, uint32_t sbits, const int8_t* hq0, float dh0, bool v0, const int8_t* hq1,
                         float dh1, bool v1) {
        const uint32_t wd[4] = {wdv.x, wdv.y, wdv.z, wdv.w};
        int ha[16];
        const int4* hp0 = reinterpret_cast<const int4*>(hq0);
        const int4* hp1 = reinterpret_cast<const int4*>(hq1);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int4 a0 = hp0[q], a1 = hp1[q];
            ha[4 * q] = a0.x;
            ha[4 * q + 1] = a0.y;
            ha[4 * q + 2] = a0.z;
            ha[4 * q + 3] = a0.w;
            ha[8 + 4 * q] = a1.x;
            ha[8 + 4 * q + 1] = a1.y;
            ha[8 + 4 * q + 2] = a1.z;
            ha[8 + 4 * q + 3] = a1.w;
        }
        int s0 = 0, s1 = 0, q0 = 0, q1 = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            q0 = dot4(int(wd[w] & 0x03030303u), ha[w], q0);
            q0 = dot4(int((wd[w] >> 2) & 0x03030303u), ha[4 + w], q0);
            q1 = dot4(int((wd[w] >> 4) & 0x03030303u), ha[8 + w], q1);
            q1 = dot4(int((wd[w] >> 6) & 0x03030303u), ha[12 + w], q1);
        }
#pragma unroll
        for (int i2 = 0; i2 < 8; ++i2) s0 = dot4(ha[i2], 0x01010101, s0);
#pragma unroll
        for (int i2 = 8; i2 < 16; ++i2) s1 = dot4(ha[i2], 0x01010101, s1);
        const float f = (v0 ? float(q0 - s0) * dh0 : 0.0f) + (v1 ? float(q1 - s1) * dh1 : 0.0f);
        return f * h2f(uint16_t(sbits));
    };
    auto own_compute = [&](int it0) {
#pragma unroll
        for (int k = 0; k < DOB; ++k) {
            const int it = it0 + tid + k * kDT;
            if (it0 + k * kDT >= nown_items) break;   // (uniform: items are whole waves)
            const bool ok = it < nown_items;
            const int itc = min(it, nown_items - 1);
            const int m = itc / (RW * NBF), rem = itc % (RW * NBF);
            const int rr = rem / NBF, c = rem % NBF;
            const int hb = m * ff + 64 * c;   // the block's h codes (pair order: entry m's rows first)
            float part = ok ? chunk_dot(dco[k], dso[k], sh_q + hb, sh_d[hb / 32], true, sh_q + hb + 32, sh_d[hb / 32 + 1], true)
                            : 0.0f;
            // the row's NBF partials in the pairwise tree of the decode kernels (lanes c of one row are
            // adjacent and aligned)
            if (NBF == 4) part = group_sum<4>(part);
            else if (NBF == 8) part = group_sum<8>(part);
            else part = group_sum<16>(part);
            if (ok && c == NBF - 1) sy[m * RW + rr] = part;
        }
    };
    auto split_compute = [&](int it) {
        const int s = it / RW, rr = it % RW;
        const int hbase = X.nown * ff + s * X.rs;   // the entry's slice in pair order
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int cc = cb0 + c;
            if (cc >= cb1) break;
            const int bA = 2 * cc, bB = 2 * cc + 1;   // the two 32-blocks of the 64-block
            const bool vA = bA >= X.hb0 && bA < X.hb1, vB = bB >= X.hb0 && bB < X.hb1;
            const int oA = hbase + (bA - X.hb0) * 32, oB = hbase + (bB - X.hb0) * 32;
            const int oAc = vA ? oA : hbase, oBc = vB ? oB : hbase;
            acc += chunk_dot(dcs[c], dss[c], sh_q + oAc, sh_d[oAc / 32], vA, sh_q + oBc, sh_d[oBc / 32], vB);
        }
        sy[(X.nown + s) * RW + rr] = acc;
    };

    FRT_D2_STAMP(4);
    if (p0 < p1) gu_load(p0);
    if (nown_items > 0 && tid < kDT) own_load(0);
    const bool has_split = tid < kDT && tid < nsplit_items && X.rs > 0;   // (an XCD may hold no block of ff < 256)
    if (has_split) split_load(tid);
    // the routing weights while the rows load (rank order: w = e / sum e, e = exp(l - l_0), the sum
    // in rank order; the shared expert's: sigmoid(gate)), then each entry's
    if (wave == 0) {
        const bool rk = lane < K;
        const float lv = rk ? R.w[0][lane] : 0.0f;
        const float e = rk ? expf(lv - R.w[0][0]) : 0.0f;
        float ws = 0.0f;
        for (int k = 0; k < K; ++k) ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), k));
        const float w = e / ws;
        if (b == 0 && rk) {
            const int id = R.ids[0][lane];
            if (a.ids) a.ids[l * K + lane] = id;
            if (a.wts) a.wts[l * K + lane] = w;
            if (a.counts) atomicAdd(a.counts + id, 1u);
        }
        const int rank = lane < U ? R.ent[lane].slot[0] : 0;
        const float wu = __shfl(w, rank < 0 ? 0 : rank);
        if (lane < K) R.ent[lane].w[0] = wu;
        if (lane == K) R.ent[K].w[0] = sigmoidf_(R.ent[K].w[0]);
    }
    for (int pb = p0; pb < p1; pb += PB * SLOTS) {
        if (pb != p0) gu_load(pb);
        gu_compute(pb);
    }
    FRT_D2_STAMP(5);
    // ---- the XCD's h values, then Q8_0 per 32 (a half-wave per block)
    __syncthreads();   // this workgroup's h values are in h_f[p0 .. p1 - 1]
    if (wave == kHPubW) {
        for (int p = p0 + lane; p < p1; p += 64) pub_local(HL + p, tag, __float_as_uint(h_f[p]));
    } else {
        constexpr int NTH = kHPubW * 64;
        wait_words_at<(kMaxPx + NTH - 1) / NTH, NTH>(
            [&](int i) { return HL + i; }, X.px, tag, deadline, errw, err_val, a.host_err,
            [&](int i, uint32_t p) {
                if (i < p0 || i >= p1) h_f[i] = __uint_as_float(p);
            }, kHPollT0);
    }
    __syncthreads();
    FRT_D2_STAMP(6);
    for (int blk = tid >> 5; blk < X.px / 32; blk += kNT2 / 32) {
        const float v = h_f[blk * 32 + (lane & 31)];
        const float am = half_max(fabsf(v));
        const float d = q8_scale(am);
        sh_q[blk * 32 + (lane & 31)] = int8_t(q8_code(v, q8_inv(d)));
        if ((lane & 31) == 0) sh_d[blk] = f16_round(d);
    }
    __syncthreads();
    // ---- down rows and this XCD's partial of each
    if (tid < kDT) {
        for (int it0 = 0; it0 < nown_items; it0 += DOB * kDT) {
            if (it0 > 0) own_load(it0);
            own_compute(it0);
        }
        if (has_split) split_compute(tid);
        for (int it = tid + kDT; X.rs > 0 && it < nsplit_items; it += kDT) {
            split_load(it);
            split_compute(it);
        }
    }
    __syncthreads();
    FRT_D2_STAMP(7);
    if (tid < RW) {
        float c = 0.0f;
        for (int m = 0; m < X.nown; ++m) c += R.ent[xcd + 8 * m].w[0] * sy[m * RW + tid];
        if (X.rs > 0)
            for (int s = 0; s < X.nsplit; ++s) c += R.ent[8 * X.nown + s].w[0] * sy[(X.nown + s) * RW + tid];
        pub(a.xp + size_t(xcd) * kD2XWords + r0 + tid, tag, __float_as_uint(c));
    }
    // ---- gather the 8 partials of rows r0 .. r0 + RW - 1, sum, publish into this XCD
    // (word i: partial i / RW of row r0 + i % RW)
    if (tid >= kXPollT0)
        wait_words_at<(8 * kMaxRW + kNT2 - kXPollT0 - 1) / (kNT2 - kXPollT0), kNT2 - kXPollT0>(
            [&](int i) { return a.xp + size_t(i / RW) * kD2XWords + r0 + i % RW; }, 8 * RW, tag, deadline, errw,
            err_val, a.host_err, [&](int i, uint32_t p) { s_part[i / RW][i % RW] = __uint_as_float(p); },
            kXPollT0);
    __syncthreads();
    FRT_D2_STAMP(8);
    const uint32_t tag_next = sync_tag(ep * uint32_t(kMaxStack) + uint32_t(l + 1));
    if (tid < RW) {
        const float o8 = ((s_part[0][tid] + s_part[1][tid]) + (s_part[2][tid] + s_part[3][tid])) +
                         ((s_part[4][tid] + s_part[5][tid]) + (s_part[6][tid] + s_part[7][tid]));
        const int row = r0 + tid;
        float o;
        if (STACK) o = xs[(row / L) * (L + 1) + row % L] + o8;
        else o = a.resid ? res + o8 : o8;
        if (l + 1 < n_layer) pub_local(XL + row, tag_next, __float_as_uint(o));
        else if (xcd == 0) a.out[row] = o;
    }
    }   // layers
    if (rs) {   // keeps the warming loads of the last layer (E > 0 always)
        float z = 0.0f;
#pragma unroll
        for (int i = 0; i < L; ++i) z += wr[i];
        if (E < 0) a.out[0] = z;
    }
    if (tid == 0) __hip_atomic_store(&a.sync->epoch[b], ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.stamps && tid == 0)
        for (int l = 0; l < n_layer; ++l)
            for (int ph = 0; ph < kD2Phases; ++ph) a.stamps[(size_t(l) * kD2Phases + ph) * G + b] = s_stamp[l][ph];
}

}  // namespace

// ---------------------------------------------------------------- host side

size_t dec1_sync_bytes();

// Shapes this kernel takes (with G workgroups, a multiple of 8): n / 64 in {16, 32, 40, 48, 64},
// ff / 64 in {4, 8, 16}, E <= 1024, K <= 32, each XCD's h values and down rows within the sync region.
static bool dec2_shape_ok(int E, int K, int n, int ff, int G) {
    const int nb = n / 64, nbf = ff / 64;
    if (E < 1 || E > 1024 || K < 1 || K > 32 || K > E) return false;
    if (n % 512 || !(nb == 16 || nb == 32 || nb == 40 || nb == 48 || nb == 64)) return false;
    if (ff % 64 || !(nbf == 4 || nbf == 8 || nbf == 16)) return false;
    if (G < 8 || G % 8 || G > kMaxGrid) return false;
    const int NL = G / 8;
    if (n % NL) return false;
    const int RW = n / NL;
    if (RW > kMaxRW || RW % 16) return false;
    const int U = K + 1, nbh = ff / 32;
    const int rs_max = 32 * ((nbh + 7) / 8);
    if ((U >> 3) * ff + (U & 7) * rs_max > kMaxPx) return false;
    return true;
}

namespace {
std::mutex g_dec2_mu;
std::set<std::pair<int, const void*>> g_dec2_init;        // (device, sync region) already zeroed
std::map<std::pair<int, const void*>, int> g_dec2_grid;   // (device, kernel) -> grid size

__global__ void k_dec2_zero(uint64_t* p, size_t words) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < words; i += size_t(gridDim.x) * blockDim.x) p[i] = 0;
}
}  // namespace

extern int g_dec1_grid_cap;
extern int g_route8;
extern uint64_t g_dec1_ticks;
int g_dec2_on = 0;   // 1: single-token calls take this kernel where it fits (else decode1.hip's)
uint64_t* g_dec2_stamps = nullptr;   // measurement only: phase stamps of the next calls (device buffer)

static int dec2_launch(Dec2Args& a, int E, int K, int n, int ff, int norm, void* sync_ws, const float* next_w,
                       hipStream_t stream, bool probe_only = false) {
    int dev = 0;
    FRT_HIP(hipGetDevice(&dev));
    uint8_t* base = static_cast<uint8_t*>(sync_ws);
    a.sync = reinterpret_cast<Dec1Sync*>(base);
    a.lg = reinterpret_cast<uint64_t*>(base + kSyncHead);
    uint64_t* t = reinterpret_cast<uint64_t*>(base + kSyncHead + kSyncLg);
    a.lgl = t;
    a.hl = a.lgl + size_t(8) * kD2LglWords;
    a.xp = a.hl + size_t(8) * kD2HlWords;
    a.xl = a.xp + size_t(8) * kD2XWords;
    a.next_w = next_w;
    a.ticks = g_dec1_ticks;
    a.stamps = g_dec2_stamps;
    a.route8 = g_route8;
    a.E = E;
    a.K = K;
    a.ff = ff;
    a.nbf = ff / 64;
    a.norm = norm;
    const int nb = n / 64;
    const bool v8 = E <= 512;
    const bool st = a.n_layer > 1;
    const void* kfn = nullptr;
#define FRT_D2PICK(NBV)                                                                                     \
    case NBV:                                                                                               \
        kfn = v8 ? (st ? reinterpret_cast<const void*>(k_dec2<NBV, 8, true>)                                \
                       : reinterpret_cast<const void*>(k_dec2<NBV, 8, false>))                              \
                 : (st ? reinterpret_cast<const void*>(k_dec2<NBV, 16, true>)                               \
                       : reinterpret_cast<const void*>(k_dec2<NBV, 16, false>));                            \
        break;
    switch (nb) {
        FRT_D2PICK(16) FRT_D2PICK(32) FRT_D2PICK(40) FRT_D2PICK(48) FRT_D2PICK(64)
        default: return kErrShape;
    }
#undef FRT_D2PICK
    int grid;
    {
        std::lock_guard<std::mutex> lk(g_dec2_mu);
        auto it = g_dec2_grid.find({dev, kfn});
        if (it == g_dec2_grid.end()) {
            // every workgroup must be resident at once: one per CU, no private (scratch) memory; the
            // largest dynamic LDS of an eligible shape must fit beside the static LDS
            int cus = 0, per_cu = 0;
            hipFuncAttributes fa{};
            FRT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
            FRT_HIP(hipFuncGetAttributes(&fa, kfn));
            const size_t smem_max = size_t(kD2HlWords) * (4 + 1) + kD2HlWords / 32 * 4 + size_t(33) * kMaxRW * 4;
            FRT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, kNT2, smem_max));
            grid = (per_cu >= 1 && cus >= 8 && fa.localSizeBytes == 0) ? (cus < kMaxGrid ? cus : kMaxGrid) : 0;
            grid -= grid % 8;
            g_dec2_grid[{dev, kfn}] = grid;
        } else {
            grid = it->second;
        }
    }
    if (g_dec1_grid_cap > 0 && g_dec1_grid_cap < grid) grid = g_dec1_grid_cap - g_dec1_grid_cap % 8;
    if (grid < 8 || !dec2_shape_ok(E, K, n, ff, grid)) return 1;   // (not this kernel)
    if (probe_only) return kOk;
    if (int rc = host_err_flag(dev, !g_dec1_no_alloc, &a.host_err)) return rc;
    {
        std::lock_guard<std::mutex> lk(g_dec2_mu);
        if (g_dec2_init.insert({dev, sync_ws}).second) {
            k_dec2_zero<<<64, 256, 0, stream>>>(reinterpret_cast<uint64_t*>(base), dec1_sync_bytes() / 8);
            FRT_LAUNCHED("decode2 zero");
        }
    }
    // dynamic LDS: the XCD's h values (floats, then int8 codes and block scales) and the down rows
    size_t smem = 0;
    {
        const int U = K + 1, nbh = ff / 32, NL = grid / 8, RW = n / NL;
        int pxm = 0;
        for (int x = 0; x < 8; ++x) {
            const int hb0 = (x * nbh) >> 3, hb1 = ((x + 1) * nbh) >> 3;
            const int px = (U >> 3) * ff + (U & 7) * 32 * (hb1 - hb0);
            pxm = px > pxm ? px : pxm;
        }
        smem = size_t(pxm) * 5 + size_t(pxm / 32) * 4 + size_t((U >> 3) + (U & 7)) * RW * 4;
    }
    const char* name = a.n_layer > 1 ? "dec2_stack" : "dec2_layer";
#define FRT_D2L(NBV, VV)                                                                              \
    if (st) launch_timed(name, k_dec2<NBV, VV, true>, dim3(grid), dim3(kNT2), smem, stream, a);       \
    else launch_timed(name, k_dec2<NBV, VV, false>, dim3(grid), dim3(kNT2), smem, stream, a);         \
    break;
#define FRT_D2N(NBV)                 \
    case NBV:                        \
        if (v8) {                    \
            FRT_D2L(NBV, 8)          \
        } else {                     \
            FRT_D2L(NBV, 16)         \
        }
    switch (nb) {
        FRT_D2N(16) FRT_D2N(32) FRT_D2N(40) FRT_D2N(48) FRT_D2N(64)
    }
#undef FRT_D2N
#undef FRT_D2L
    FRT_LAUNCHED("decode2 layer");
    return kOk;
}

// 1 when a single-token layer (stack: n_layer > 1) of this shape runs in this kernel.
int dec2_support(int E, int K, int n, int ff, int n_layer) {
    if (!g_dec2_on) return 0;
    Dec2Args a{};
    a.n_layer = n_layer;
    return dec2_launch(a, E, K, n, ff, 0, nullptr, nullptr, nullptr, true) == kOk ? 1 : 0;
}

int dec2_layer(const float* x, const float* W, const float* bias, const float* gate_w, int E, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared, int n, int ff, int norm, const float* resid,
               float* out, int32_t* ids, float* wts, uint32_t* counts, void* sync_ws, const float* next_w,
               hipStream_t stream) {
    Dec2Args a{};
    a.lay[0] = Dec1Layer{W, bias, gate_w, arena, shared};
    a.n_layer = 1;
    a.x = x;
    a.stride = stride;
    a.resid = resid;
    a.out = out;
    a.ids = ids;
    a.wts = wts;
    a.counts = counts;
    const int rc = dec2_launch(a, E, K, n, ff, norm, sync_ws, next_w, stream);
    return rc == 1 ? set_error(kErrShape, "decode2: shape") : rc;
}

int dec2_stack(const frt_moe_layer* L, int n_layer, const float* x, float* out, int32_t* ids, float* wts,
               void* sync_ws, hipStream_t stream) {
    if (n_layer < 1 || n_layer > kMaxStack) return set_error(kErrShape, "decode2 stack: %d layers (1..%d)", n_layer, kMaxStack);
    Dec2Args a{};
    for (int l = 0; l < n_layer; ++l)
        a.lay[l] = Dec1Layer{L[l].router_w, L[l].router_bias, L[l].gate_w, L[l].experts, L[l].shared};
    a.n_layer = n_layer;
    a.x = x;
    a.stride = L[0].stride;
    a.out = out;
    a.ids = ids;
    a.wts = wts;
    const int norm = (L[0].flags & FRT_LAYER_NORM_INPUT) ? 1 : 0;
    if (n_layer == 1) a.resid = x;
    const int rc = dec2_launch(a, L[0].n_expert, L[0].top_k, L[0].d_model, L[0].d_ff, norm, sync_ws,
                               L[n_layer - 1].next_router_w, stream);
    return rc == 1 ? set_error(kErrShape, "decode2: shape") : rc;
}

}  // namespace frt
