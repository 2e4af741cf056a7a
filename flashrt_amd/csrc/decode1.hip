// Single-token MoE layer (T = 1 decode) as ONE persistent launch.
//
// The three dependent steps of a decode layer (router logits -> routing + gate/up -> down +
// combine; moe_block_fast, arch/qwen4exp/moe_fast.cu:1015-1108, and the phase A / phase B split of
// quant/q2_0/moe_cpu.cpp:36-114) run in one grid of one 512-thread workgroup per CU, all resident
// together, joined inside the kernel rather than by kernel boundaries:
//   1. router: every workgroup stages x in LDS, forms the canonical RMS scale, computes its router
//      rows (one wave per row, the canonical order of route.hip) and publishes the logits; it also
//      quantizes the experts' input (Q8_0 per 32) into its own LDS.
//   2. routing + gate/up: every workgroup waits for all E + 1 logits (the shared gate last), routes
//      the token itself (route1_wave), issues the gate/up rows of its unit (entry x 32 ff rows) and,
//      behind them (waves 0-3), the down rows of its 8 output rows for every entry (those land while
//      the gate/up work and the wait below run); each row's block terms are added in the CPU path's
//      order (seq_row_sums); SwiGLU and Q8_0 of the 32-row h block, published.
//   3. down: every workgroup waits for all h blocks (polled by waves 4-7, whose waits do not queue
//      behind down-row loads), finishes its down rows and the combine, the same float order as
//      k_dec_down's single-token combine (outputs equal the three-kernel path's bit for bit).
//
// Joins: epoch-tagged 8-byte words, (tag << 32) | payload, stored and loaded at agent scope (sc1),
// so that a reader on another XCD sees the writer's value and never a stale line of its own L2.
// tag = f(epoch). Each workgroup keeps an epoch cell at the front of the workspace; at its start it
// reads every cell and takes the largest + 1, at its end it stores that in its own cell. No cell is
// stored before every workgroup has read them all (a workgroup stores only after it has seen every
// workgroup's logits, published after that workgroup read the cells), so all workgroups of a call
// agree on the epoch even over cells that hold anything, and each call's epoch exceeds every epoch
// stored before it; a word is current exactly when its tag
// matches: no flag, fence or counter is needed, and no late word of one call can pass for the next
// call's. Every wait is bounded by ticks of the 100 MHz constant clock
// (20M by default) for the whole call: past it the call sets the error word and finishes with what it read, so a
// workgroup that never became resident cannot hang the GPU.
#include <hip/hip_runtime.h>

// In this file threadIdx.x is read through an empty volatile asm: values derived from it are then
// computed where they are used rather than hoisted out of the stack kernel's layer loop, which kept
// dozens of per-thread addresses live across the whole loop and spilled registers.
struct FrtOpaqueTid {
    __device__ unsigned get_x() const {
        unsigned t = __builtin_amdgcn_workitem_id_x();
        asm volatile("" : "+v"(t));
        return t;
    }
    __declspec(property(get = get_x)) unsigned x;
};
#define threadIdx (FrtOpaqueTid{})
#include "decode_parts.hpp"
#include "persist.hpp"

#include "../../include/flashrt_moe.h"

#include <map>
#include <mutex>
#include <set>
#include <utility>

namespace frt {

// Words between two published words of the logits, h blocks and x: every workgroup polls every
// word, pollers of one line queue on it, and more lines mean more requests (measured: 4 / 1 / 1).
constexpr int kLgStride = 4;
constexpr int kHbStride = 1;
constexpr int kXbStride = 1;

namespace {

constexpr int kNT1 = kNTP;         // threads per workgroup
constexpr int kNW1 = kNT1 / 64;    // waves per workgroup
constexpr int kMaxHWords = 8 * kNT1;   // h words one call can publish (8 per thread to wait for)

struct Dec1Args {
    Dec1Layer lay[kMaxStack];
    int n_layer;           // 1: one layer (resid optional); more: a stack, x_{l+1} = x_l + moe_l(x_l)
    const float* x;        // [n] the (first) layer's input
    size_t stride;
    const float* resid;    // [n] or null (one layer)
    float* out;            // [n] the (last) layer's output
    int32_t* ids;          // [n_layer][K] rank order, or null
    float* wts;            // [n_layer][K], or null
    uint32_t* counts;      // [E] or null (one layer)
    uint64_t* xb;          // [n] tagged words of the next layer's input (a stack)
    Dec1Sync* sync;
    uint64_t* lg;          // [E + 1] tagged logits (the shared gate last), one per 128-byte line (kLgStride words)
    uint64_t* hb;          // [U * ff/32][9] tagged h blocks: 8 words of 4 codes, then the scale
    const float* next_w;   // the next layer's router [E][n] (cache warming) or null
    uint64_t ticks;        // bound of the call's waits, in ticks of the 100 MHz constant clock
    uint32_t* host_err;    // host-visible flag set with the error word (pinned host memory), or null
    int route8;            // the single-token routing by all 8 waves (route_8waves) rather than one
    int E, K, ff, norm;
};

typedef const __attribute__((address_space(4))) Dec1Args KArgs;
typedef const __attribute__((address_space(4))) Dec1Layer KLayer;

template <int PASSES>
struct Dec1Lds {
    WinLds R;
    float s_h[32];
    Route8Lds q8;
    __align__(16) float seq[kNW1][PASSES * 128];   // per wave: the gate/up block terms of seq_row_sums
};

template <int NB, int V, int NBF, bool STACK>
__global__ void __launch_bounds__(kNT1) k_dec1(Dec1Args a_byval) {
    // the arguments are read where they lie (the kernel argument segment, scalar loads): indexing
    // the layer table of a by-value copy would place the whole block in private memory
    (void)a_byval;
    const KArgs& a = *(const KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int n = 64 * NB, L = NB;   // the router's 64 chains are L = n / 64 long
    extern __shared__ __align__(16) uint8_t smem[];   // sh_q [U][ff] | sh_d [U][ff/32] | sh_y [U][8]
    __shared__ float xs[64 * (L + 1)];                // x by chain, each chain padded by one float
    __shared__ __align__(16) int8_t xq[n];
    __shared__ float xd[n / kQ8];
    __shared__ __align__(16) float s_lg[64 * V + 4];
    __shared__ Dec1Lds<gu_passes<NB, kNW1>()> S;
    WinLds& R = S.R;

    const int b = blockIdx.x, G = gridDim.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = a.E, K = a.K, ff = a.ff, U = K + 1, RB = ff / 32, NU = U * RB;
    const uint64_t deadline = wall_clock64() + a.ticks;
    // the epoch: the largest cell + 1 (cells read one per thread; the maximum after the first barrier)
    __shared__ uint32_t s_ep[kNW1];
    {
        uint32_t c = tid < G ? __hip_atomic_load(&a.sync->epoch[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        if (G > kNT1)
            for (int i = tid + kNT1; i < G; i += kNT1)
                c = max(c, __hip_atomic_load(&a.sync->epoch[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        for (int o = 32; o > 0; o >>= 1) c = max(c, uint32_t(__shfl_xor(int(c), o, 64)));
        if (lane == 0) s_ep[wave] = c;
    }

    // ---- 1. router rows (slot s = b + G w for wave w; slot E is the shared gate row), then x
    const int s0 = b + wave * G;
    const bool rs = s0 <= E;
    float wr[L];
    float bias_v = 0.0f;
    auto load_router = [&](const KLayer& LY) {
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
        bias_v = LY.bias ? LY.bias[min(s0, E - 1)] : 0.0f;
    };
    load_router(a.lay[0]);
    constexpr int XV = (n / 4 + kNT1 - 1) / kNT1;
    float4 xv[XV];
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
#pragma unroll
    for (int k = 0; k < XV; ++k) xv[k] = x4[min(tid + k * kNT1, n / 4 - 1)];
    const int r0 = 8 * b;   // this workgroup's first down row group
    const float res = a.resid ? a.resid[min(r0 + (tid & 7), n - 1)] : 0.0f;
#pragma unroll
    for (int k = 0; k < XV; ++k) {
        const int idx = tid + k * kNT1;
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
    for (int w = 1; w < kNW1; ++w) ep = max(ep, s_ep[w]);
    ep += 1u;
    constexpr bool stack = STACK;
    const uint64_t err_val = (uint64_t(kErrMagic) << 32) | ep;
    const int n_layer = STACK ? a.n_layer : 1;
    for (int l = 0; l < n_layer; ++l) {
    const KLayer& LY = a.lay[l];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;   // per layer (see FrtOpaqueTid)
    const uint32_t tag = sync_tag(ep * uint32_t(kMaxStack) + uint32_t(l));
    if (l > 0) {   // x_l from the previous layer's down rows
        load_router(LY);   // rows warmed into this XCD's L2 by the previous layer: they land during the wait
        __syncthreads();   // the previous combine has read xs
        wait_words<(64 * 64 + kNT1 - 1) / kNT1, kXbStride>(a.xb, n, tag, deadline, &a.sync->err, err_val, a.host_err,
                                                [&](int i, uint32_t p) { xs[(i / L) * (L + 1) + i % L] = __uint_as_float(p); });
        __syncthreads();
    }
    const float r = a.norm ? rms_scale_wave<L>(xs + lane * (L + 1), n) : 1.0f;
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
        if (lane == 0) pub(a.lg + size_t(s) * kLgStride, tag, __float_as_uint(acc));
    };
    if (rs) router_dot(s0, wr, bias_v);
    for (int s = s0 + kNW1 * G; s <= E; s += kNW1 * G) {   // only with fewer than (E + 1) / 8 workgroups
        float w2[L];
        const float* wrow = s < E ? LY.W + size_t(s) * n : LY.gate_w;
#pragma unroll
        for (int i = 0; i < L; ++i) w2[i] = wrow[lane * L + i];
        router_dot(s, w2, LY.bias && s < E ? LY.bias[s] : 0.0f);
    }
    // Q8_0 of the experts' input (u = x r with the norm) by the last two waves, which hold no router
    // row (with one workgroup per CU, (E + 1) / G < 6): a lane pair per 32-block, 16 values a lane
    if (wave >= kNW1 - 2) {
        const int h = lane & 1;
        for (int b0 = (wave - (kNW1 - 2)) * 32; b0 < n / kQ8; b0 += 64) {   // the same count in both waves' lanes
            const int blk = min(b0 + (lane >> 1), n / kQ8 - 1);
            float v[16];
            float am = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int k = blk * kQ8 + 16 * h + j;
                v[j] = xs[(k / L) * (L + 1) + k % L];
                if (a.norm) v[j] = v[j] * r;
                am = fmaxf(am, fabsf(v[j]));
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

    // ---- 2. all logits, the routing, gate/up
    wait_words<(1024 + 1 + kNT1 - 1) / kNT1, kLgStride>(a.lg, E + 1, tag, deadline, &a.sync->err, err_val, a.host_err,
                                            [&](int i, uint32_t p) { s_lg[i] = __uint_as_float(p); });
    if (E <= 512 && a.route8) {   // the 8 waves route together (each may start on its own logits)
        route_8waves(s_lg, E, K, LY.arena, a.stride, LY.shared, R, S.q8);
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
    __syncthreads();
    if (R.many) {   // more than 64 candidates (heavily tied logits): four waves select, as window_entries
        float mx;
        topk_group4<V>(s_lg, E, K, wave & 3, wave < 4, R.tk[0], mx);
        if (wave == 0) {
            const float sel_l = lane < K ? R.tk[0].sel_v[lane] : 0.0f;
            const int sel_id = lane < K ? R.tk[0].sel_id[lane] : 0x7fffffff;
            int u = 0;
            for (int j = 0; j < K; ++j) u += int(__builtin_amdgcn_readlane(sel_id, j) < sel_id);
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

    // gate/up unit q = b + i G: entry q / RB, ff rows 32 (q % RB) .. + 31; 32 / kNW1 rows per wave
    constexpr int RPW = gu_rpw<NB>();   // rows per wave pass
    constexpr int ROWS = 32 / kNW1;
    constexpr int PASSES = gu_passes<NB, kNW1>();
    const int rsub = lane / NB, bk = lane % NB;
    const bool live = rsub < RPW;
    const int bl = live ? bk : 0;
    const size_t mb = mat_bytes(ff, n);
    uint4 cg[PASSES], cu[PASSES];
    uint32_t sg[PASSES], su[PASSES];
    uint32_t okm = 0;
    auto gu_load = [&](int q) {
        const DecEntry& e = R.ent[q / RB];
        const int rb = q % RB;
        const uint8_t* gcodes = e.blob;
        const uint16_t* gscal = reinterpret_cast<const uint16_t*>(e.blob + size_t(ff) * NB * 16);
        const uint8_t* ucodes = e.blob + mb;
        const uint16_t* uscal = reinterpret_cast<const uint16_t*>(e.blob + mb + size_t(ff) * NB * 16);
        okm = 0;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int rl = p * RPW + rsub;
            if (live && rl < ROWS) okm |= 1u << p;
            const int row = rb * 32 + wave * ROWS + min(rl, ROWS - 1);
            cg[p] = gld_u4_nt(gcodes + (size_t(row) * NB + bl) * 16);
            cu[p] = gld_u4_nt(ucodes + (size_t(row) * NB + bl) * 16);
            sg[p] = gld<uint16_t>(gscal + size_t(row) * NB + bl);
            su[p] = gld<uint16_t>(uscal + size_t(row) * NB + bl);
        }
    };
    auto gu_compute = [&](int q) {
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
        float tg[PASSES], tu[PASSES];
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const uint32_t wg[4] = {cg[p].x, cg[p].y, cg[p].z, cg[p].w};
            const uint32_t wu[4] = {cu[p].x, cu[p].y, cu[p].z, cu[p].w};
            const bool okp = (okm >> p) & 1u;
            const float dg = okp ? h2f(uint16_t(sg[p])) : 0.0f, du = okp ? h2f(uint16_t(su[p])) : 0.0f;
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
            tg[p] = fg * dg;
            tu[p] = fu * du;
        }
        // the rows' sums over their NB lanes in the CPU path's order, all passes at once: lane
        // 2 RPW p + r holds row p RPW + r
        const float2 gu = seq_row_sums<NB, RPW, PASSES>(tg, tu, S.seq[wave], lane);
        {
            const int p = lane / (2 * RPW), r = lane % (2 * RPW), row = p * RPW + r;
            if (r < RPW && p < PASSES && row < ROWS) S.s_h[wave * ROWS + row] = gu.x / (1.0f + expf(-gu.x)) * gu.y;
        }
        __syncthreads();
        if (wave == 0) {   // Q8_0 of the 32-row h block, published as 8 words of 4 codes and the scale
            const float v = lane < 32 ? S.s_h[lane] : 0.0f;
            const float am = half_max(fabsf(v));
            const float d = q8_scale(am);
            const int c = q8_code(v, q8_inv(d)) & 0xff;
            const int l4 = (4 * lane) & 63;
            const uint32_t word = uint32_t(__shfl(c, l4)) | (uint32_t(__shfl(c, l4 + 1)) << 8) |
                                  (uint32_t(__shfl(c, l4 + 2)) << 16) | (uint32_t(__shfl(c, l4 + 3)) << 24);
            uint64_t* dst = a.hb + size_t(q) * 9 * kHbStride;
            if (lane < 8) pub(dst + lane * kHbStride, tag, word);
            if (lane == 8) pub(dst + 8 * kHbStride, tag, __float_as_uint(f16_round(d)));
        }
    };

    const bool has_down = r0 < n;
    if (b < NU) gu_load(b);
    // the routing weights while the rows load (rank order: w = e / sum e, e = exp(l - l_0), the
    // sum in rank order; the shared expert's: sigmoid(gate)), then each entry's
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
    for (int q = b; q < NU; q += G) {
        if (q != b) {
            __syncthreads();   // wave 0 has read s_h of the previous unit
            gu_load(q);
        }
        gu_compute(q);
    }

    // ---- 3. all h blocks, then the down rows and the combine
    int8_t* sh_q = reinterpret_cast<int8_t*>(smem);
    float* sh_d = reinterpret_cast<float*>(smem + size_t(U) * ff);
    float* sh_y = sh_d + size_t(U) * (ff / kQ8);
    // warm this XCD's L2 with the next layer's router rows this workgroup will read (issued ahead of
    // the wait, which they would otherwise only delay at the kernel's end)
    // the down rows of this workgroup's 8 output rows for every entry (the first 12 entries), issued
    // once the gate/up rows no longer compete with them; they land during the wait below. Loaded
    // by waves 0-3 (entries wave + 4 i); waves 4-7 poll the h words meanwhile. A wave's waits count its
    // loads in issue order, so a poller that had issued down rows would wait behind them (measured on
    // the stack: all waves loading and polling 722-733 us per token, split 705-714)
    DownRegs<NBF, 3> D3;
    if (has_down && wave < 4) down_load<NBF, 3, 4, true>(R.ent, U, wave, r0, n, ff, D3);
    // warm this XCD's L2 with the router rows this workgroup reads next: the next layer's (a stack),
    // else the next call's
    const float* warm_w = l + 1 < n_layer ? a.lay[l + 1].W : a.next_w;
    float4 nv[L / 4];
    const bool warm = warm_w && rs && s0 < E;
    if (warm) {
        const float4* w4 = reinterpret_cast<const float4*>(warm_w + size_t(s0) * n + lane * L);
#pragma unroll
        for (int i = 0; i < L / 4; ++i) nv[i] = w4[i];
    }
    {   // the first kHPoll words by waves 4-7, any beyond by waves 0-3 (shapes with many h blocks)
        constexpr int kHPoll = 8 * (kNT1 / 2);
        auto put_h = [&](int i, uint32_t p) {
            const int q = i / 9, part = i % 9, u = q / RB, rb = q % RB;
            if (part < 8) *reinterpret_cast<uint32_t*>(sh_q + size_t(u) * ff + rb * 32 + 4 * part) = p;
            else sh_d[u * (ff / kQ8) + rb] = __uint_as_float(p);
        };
        const int nh = NU * 9;
        if (wave >= kNW1 / 2)
            wait_words_at<8, kNT1 / 2>([&](int i) { return a.hb + size_t(i) * kHbStride; }, min(nh, kHPoll), tag, deadline,
                                       &a.sync->err, err_val, a.host_err, put_h, kNT1 / 2);
        else if (nh > kHPoll)
            wait_words_at<8, kNT1 / 2>([&](int i) { return a.hb + size_t(kHPoll + i) * kHbStride; }, nh - kHPoll, tag,
                                       deadline, &a.sync->err, err_val, a.host_err,
                                       [&](int i, uint32_t p) { put_h(kHPoll + i, p); }, 0);
    }
    __syncthreads();
    // combine of rows g0 .. g0 + 7 (threads 0..7): the routed entries in ascending expert id from 0,
    // then the shared expert, then the residual (k_dec_down's single-token order)
    // (a stack adds the layer's input x_l and hands the row to the next layer as a tagged word)
    const uint32_t tag_next = sync_tag(ep * uint32_t(kMaxStack) + uint32_t(l + 1));
    auto combine = [&](int g0, float rv) {
        if (tid < 8) {
            float acc = 0.0f;
            for (int u = 0; u < K; ++u) {
                const float p = R.ent[u].w[0] * sh_y[u * 8 + tid];
                acc = acc + p;
            }
            float o = acc + sh_y[K * 8 + tid] * R.ent[K].w[0];
            const int row = g0 + tid;
            if (stack) o = xs[(row / L) * (L + 1) + row % L] + o;
            else if (a.resid) o = rv + o;
            if (l + 1 < n_layer) pub(a.xb + size_t(row) * kXbStride, tag_next, __float_as_uint(o));
            else a.out[row] = o;
        }
    };
    if (has_down) {
        if (wave < 4) {
            down_compute1<NBF, 3, 4>(U, wave, D3, sh_q, sh_d, sh_y, ff);
            for (int u0 = wave + 12; u0 < U; u0 += 12) {
                DownRegs<NBF, 3> D2;
                down_load<NBF, 3, 4, true>(R.ent, U, u0, r0, n, ff, D2);
                down_compute1<NBF, 3, 4>(U, u0, D2, sh_q, sh_d, sh_y, ff);
            }
        }
        __syncthreads();
        combine(r0, res);
    }
    for (int g0 = r0 + 8 * G; g0 < n; g0 += 8 * G) {   // more 8-row groups than workgroups
        const float rv = (!stack && a.resid) ? a.resid[g0 + (tid & 7)] : 0.0f;
        __syncthreads();   // sh_y of the previous group is combined
        constexpr int MB = 2;   // entries per wave and batch (all waves: h is in LDS by now)
        for (int u0 = wave; u0 < U; u0 += kNW1 * MB) {
            DownRegs<NBF, MB> D2;
            down_load<NBF, MB, kNW1, true>(R.ent, U, u0, g0, n, ff, D2);
            down_compute<NBF, MB, kNW1>(R.ent, U, u0, D2, sh_q, sh_d, sh_y, ff);
        }
        __syncthreads();
        combine(g0, rv);
    }
    if (warm) {   // keeps the warming loads (E > 0 always)
        float z = 0.0f;
#pragma unroll
        for (int i = 0; i < L / 4; ++i) z += nv[i].x + nv[i].y + nv[i].z + nv[i].w;
        if (E < 0) a.out[0] = z;
    }
    }   // layers
    if (tid == 0) __hip_atomic_store(&a.sync->epoch[b], ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_dec1_zero(uint64_t* p, size_t words) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < words; i += size_t(gridDim.x) * blockDim.x) p[i] = 0;
}

}  // namespace

// ---------------------------------------------------------------- host side

// The sync region at the front of every layer workspace: the error word and the epoch cells, then
// the tagged words (sized for the largest eligible call: E <= 1024, 4096 h words).
constexpr size_t kDec1Head = kSyncHead;
constexpr size_t kDec1Lg = kSyncLg;   // room for any logit stride up to 16
constexpr size_t kDec1Hb = size_t(kMaxHWords) * 8 * kHbStride;
constexpr size_t kDec1Xb = size_t(64 * 64) * 8 * kXbStride;   // a stack's next-layer input, n <= 4096
// (decode2.hip's words follow the logits in the same region; both kernels share the epoch cells)
size_t dec1_sync_bytes() { return kDec1Head + kDec1Lg + (kDec1Hb + kDec1Xb > kD2Tail ? kDec1Hb + kDec1Xb : kD2Tail); }

int dec1_eligible(int E, int K, int n, int ff) {
    const int nb = n / 64, nbf = ff / 64;
    if (E < 1 || E > 1024 || K < 1 || K > 32 || K > E) return 0;
    if (n % 512 || !(nb == 16 || nb == 32 || nb == 40 || nb == 48 || nb == 64)) return 0;
    if (ff % 64 || !(nbf == 4 || nbf == 8 || nbf == 10 || nbf == 16)) return 0;
    if ((K + 1) * (ff / 32) * 9 > kMaxHWords) return 0;
    return 1;
}

constexpr int kErrUnfit = 1;   // internal: the persistent kernel cannot run this shape

namespace {
std::mutex g_dec1_mu;
std::set<std::pair<int, const void*>> g_dec1_init;   // (device, sync region) already zeroed
std::map<std::pair<int, const void*>, int> g_dec1_grid;   // (device, kernel) -> grid size
}  // namespace

// The host-visible time-out flag of each device: pinned, mapped host memory that a persistent call
// whose wait ran out of time sets (a system-scope store) beside the workspace's error word, so that
// the next call through the C ABI reports it without synchronising (kErrSync). Allocated at the
// first persistent launch on a device; an allocation-free call only uses it once it exists.
namespace {
constexpr int kMaxDev = 64;
std::mutex g_herr_mu;
uint32_t* g_herr_host[kMaxDev] = {};
uint32_t* g_herr_dev[kMaxDev] = {};
}  // namespace

int host_err_flag(int dev, bool may_alloc, uint32_t** dptr) {
    *dptr = nullptr;
    if (dev < 0 || dev >= kMaxDev) return kOk;
    std::lock_guard<std::mutex> lk(g_herr_mu);
    if (!g_herr_host[dev] && may_alloc) {
        void* h = nullptr;
        FRT_HIP(hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent));
        void* d = nullptr;
        FRT_HIP(hipHostGetDevicePointer(&d, h, 0));
        *static_cast<volatile uint32_t*>(h) = 0u;
        g_herr_host[dev] = static_cast<uint32_t*>(h);
        g_herr_dev[dev] = static_cast<uint32_t*>(d);
    }
    *dptr = g_herr_dev[dev];
    return kOk;
}

// kErrSync (and clears the flag) if a persistent call on the current device ran out of time since the
// last check; no synchronisation (the flag is read where the GPU wrote it, in host memory).
int dec1_take_timeout() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return kOk;
    uint32_t* h;
    {
        std::lock_guard<std::mutex> lk(g_herr_mu);
        h = g_herr_host[dev];
    }
    if (!h) return kOk;
    volatile uint32_t* v = h;
    if (*v == 0u) return kOk;
    *v = 0u;
    return set_error(kErrSync, "a persistent decode call on device %d ran out of time waiting for another workgroup; "
                               "its outputs are undefined", dev);
}
static void host_err_clear() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return;
    std::lock_guard<std::mutex> lk(g_herr_mu);
    if (g_herr_host[dev]) *static_cast<volatile uint32_t*>(g_herr_host[dev]) = 0u;
}
// set by the allocation-free entry point around its call: no allocation of the flag then
thread_local bool g_dec1_no_alloc = false;

// Whether the next decode calls take this path (1, the default) or the three-kernel one (0), and
// the bound of a call's waits (200 ms of the 100 MHz constant clock by default).
int g_dec1_on = 1;
uint64_t g_dec1_ticks = 20000000ull;
int g_dec1_grid_cap = 0;   // workgroups per call (0: one per CU)
int g_route8 = 0;          // single-token routing by the workgroup's 8 waves (1) or by one wave (0, measured faster)

// Launches the persistent kernel for a filled-in argument block (layers, input and outputs).
// Returns kErrUnfit (no error message) when the kernel for this shape cannot have every workgroup
// resident; probe_only: only that check, no launch.
static int dec1_launch(Dec1Args& a, int E, int K, int n, int ff, int norm, void* sync_ws, const float* next_w,
                       hipStream_t stream, bool probe_only = false) {
    if (!dec1_eligible(E, K, n, ff)) return set_error(kErrShape, "decode1: E=%d K=%d n=%d ff=%d", E, K, n, ff);
    int dev = 0;
    FRT_HIP(hipGetDevice(&dev));
    uint8_t* base = static_cast<uint8_t*>(sync_ws);
    a.sync = reinterpret_cast<Dec1Sync*>(base);
    a.lg = reinterpret_cast<uint64_t*>(base + kDec1Head);
    a.hb = reinterpret_cast<uint64_t*>(base + kDec1Head + kDec1Lg);
    a.xb = reinterpret_cast<uint64_t*>(base + kDec1Head + kDec1Lg + kDec1Hb);
    a.next_w = next_w;
    a.ticks = g_dec1_ticks;
    a.route8 = g_route8;
    if (!probe_only)
        if (int rc = host_err_flag(dev, !g_dec1_no_alloc, &a.host_err)) return rc;
    a.E = E;
    a.K = K;
    a.ff = ff;
    a.norm = norm;
    if (!probe_only) {
        // a sync region not seen before is zeroed first: the epochs agree over any cell contents, but
        // leftover words could by chance carry the next call's tag
        std::lock_guard<std::mutex> lk(g_dec1_mu);
        if (g_dec1_init.insert({dev, sync_ws}).second) {
            k_dec1_zero<<<64, 256, 0, stream>>>(reinterpret_cast<uint64_t*>(base), dec1_sync_bytes() / 8);
            FRT_LAUNCHED("decode1 zero");
        }
    }
    const int U = K + 1;
    const size_t smem = size_t(U) * ff + size_t(U) * (ff / kQ8) * 4 + size_t(U) * 8 * 4;
    const void* kfn = nullptr;
    auto launch = [&](auto kern) -> int {
        kfn = reinterpret_cast<const void*>(kern);
        int grid;
        {
            std::lock_guard<std::mutex> lk(g_dec1_mu);
            auto it = g_dec1_grid.find({dev, kfn});
            if (it == g_dec1_grid.end()) {
                // every workgroup must be resident at once: one per CU, the kernel must fit, and it
                // must need no private (scratch) memory, whose allocation could hold workgroups back
                int cus = 0, per_cu = 0;
                hipFuncAttributes fa{};
                FRT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
                FRT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNT1, smem));
                FRT_HIP(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kern)));
                grid = (per_cu >= 1 && cus >= 1 && fa.localSizeBytes == 0) ? (cus < kMaxGrid ? cus : kMaxGrid) : 0;
                g_dec1_grid[{dev, kfn}] = grid;
            } else {
                grid = it->second;
            }
        }
        if (grid < 1) return kErrUnfit;
        if (g_dec1_grid_cap > 0 && g_dec1_grid_cap < grid) grid = g_dec1_grid_cap;
        if (probe_only) return kOk;
        launch_timed(a.n_layer > 1 ? "dec1_stack" : "dec1_layer", kern, dim3(grid), dim3(kNT1), smem, stream, a);
        FRT_LAUNCHED("decode1 layer");
        return kOk;
    };
    const int nb = n / 64, nbf = ff / 64;
    const bool v8 = E <= 512;
    const bool st = a.n_layer > 1;
#define FRT_D1S(NBV, VV, NBFV) \
    return st ? launch(k_dec1<NBV, VV, NBFV, true>) : launch(k_dec1<NBV, VV, NBFV, false>);
#define FRT_D1F(NBV, VV)                       \
    switch (nbf) {                             \
        case 4: FRT_D1S(NBV, VV, 4)            \
        case 8: FRT_D1S(NBV, VV, 8)            \
        case 10: FRT_D1S(NBV, VV, 10)          \
        case 16: FRT_D1S(NBV, VV, 16)          \
    }                                          \
    break;
#define FRT_D1N(NBV)              \
    case NBV:                     \
        if (v8) {                 \
            FRT_D1F(NBV, 8)       \
        } else {                  \
            FRT_D1F(NBV, 16)      \
        }                         \
        break;
    switch (nb) {
        FRT_D1N(16) FRT_D1N(32) FRT_D1N(40) FRT_D1N(48) FRT_D1N(64)
    }
#undef FRT_D1N
#undef FRT_D1F
#undef FRT_D1S
    return set_error(kErrShape, "decode1: n=%d ff=%d", n, ff);
}

int dec1_layer(const float* x, const float* W, const float* bias, const float* gate_w, int E, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared, int n, int ff, int norm, const float* resid,
               float* out, int32_t* ids, float* wts, uint32_t* counts, void* sync_ws, const float* next_w,
               hipStream_t stream) {
    Dec1Args a{};
    a.lay[0] = Dec1Layer{W, bias, gate_w, arena, shared};
    a.n_layer = 1;
    a.x = x;
    a.stride = stride;
    a.resid = resid;
    a.out = out;
    a.ids = ids;
    a.wts = wts;
    a.counts = counts;
    return dec1_launch(a, E, K, n, ff, norm, sync_ws, next_w, stream);
}

// A stack of single-token layers in one launch: x_{l+1} = x_l + moe_l(x_l), out = x_L.
int dec1_stack(const frt_moe_layer* L, int n_layer, const float* x, float* out, int32_t* ids, float* wts,
               void* sync_ws, hipStream_t stream) {
    if (n_layer < 1 || n_layer > kMaxStack) return set_error(kErrShape, "decode1 stack: %d layers (1..%d)", n_layer, kMaxStack);
    Dec1Args a{};
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
    return dec1_launch(a, L[0].n_expert, L[0].top_k, L[0].d_model, L[0].d_ff, norm, sync_ws,
                       L[n_layer - 1].next_router_w, stream);
}

// The last single-token call's logits in a sync region: logit e at the returned pointer + e * stride
// (the payload half of each tagged word).
const float* dec1_logits(const void* sync_ws, int* stride_floats) {
    *stride_floats = 2 * kLgStride;
    return reinterpret_cast<const float*>(static_cast<const uint8_t*>(sync_ws) + kDec1Head);
}

// Whether the persistent kernels can run this shape: 2 = the stack kernel too, 1 = single layers only, 0 = none.
int dec1_support(int E, int K, int n, int ff) {
    if (!dec1_eligible(E, K, n, ff)) return 0;
    Dec1Args a{};
    a.n_layer = 1;
    if (dec1_launch(a, E, K, n, ff, 0, nullptr, nullptr, nullptr, true) != kOk) return 0;
    a.n_layer = 2;
    return dec1_launch(a, E, K, n, ff, 0, nullptr, nullptr, nullptr, true) == kOk ? 2 : 1;
}

// Reads and clears the error word of a sync region (synchronous; for tests and harnesses).
int dec1_status(void* sync_ws, hipStream_t stream, uint32_t* err) {
    uint64_t e = 0;
    FRT_HIP(hipMemcpyAsync(&e, static_cast<uint8_t*>(sync_ws) + offsetof(Dec1Sync, err), 8, hipMemcpyDeviceToHost,
                           stream));
    FRT_HIP(hipStreamSynchronize(stream));
    *err = uint32_t(e >> 32) == kErrMagic ? 1u : 0u;
    host_err_clear();   // reported here: the next call need not report it again
    if (e) {
        const uint64_t z = 0;
        FRT_HIP(hipMemcpyAsync(static_cast<uint8_t*>(sync_ws) + offsetof(Dec1Sync, err), &z, 8, hipMemcpyHostToDevice,
                               stream));
        FRT_HIP(hipStreamSynchronize(stream));
    }
    return kOk;
}

}  // namespace frt
