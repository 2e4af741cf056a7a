// Decode windows of 2-4 tokens (speculative verify batches, configs[1]) as ONE persistent launch.
//
// The window path of decode.hip runs a window as four launches (router + Q8_0, routing and grouping
// in one workgroup, gate/up per entry, down + combine). This kernel runs the same steps in one grid
// of one 512-thread workgroup per CU, all resident, joined by epoch-tagged words as k_dec1
// (decode1.hip) joins a single token's (moe_hits over a window, moe_fast.cu:195-355, 498-576; the
// reference reads each distinct expert once per window):
//   1. router: every workgroup stages the T tokens' inputs, forms each token's canonical RMS scale,
//      computes its router rows for all T tokens (one wave per row, route.hip's canonical order) and
//      publishes the T logits of each row; then the workgroup quantizes the T inputs (Q8_0 per 32)
//      into its LDS.
//   2. routing + gate/up: every workgroup waits for the T (E + 1) logits, routes token t with wave t
//      (topk_wave_fast, k_win_route's selection), groups the (token, slot) items into entries of at
//      most 4 tokens per distinct expert (the shared one included) in order of first appearance, as
//      k_win_route does,
//      and forms each token's combine list (its routed slots in ascending expert id, then the shared
//      one). Unit q = b + i G: entry q / RB, ff rows 32 (q % RB) .. + 31, for every token of the
//      entry; SwiGLU and Q8_0 of each token's 32-row h block, published as 9 words.
//   3. down: every workgroup waits for all h blocks, computes its 8 output rows for every (entry,
//      token) slot (down_load / down_compute) and the combine of each token (ascending expert id from
//      0, then the shared expert, then the residual; moe_cpu.cpp:63-80).
// Every wait is bounded as in k_dec1 (the error word, the host-visible flag).
#include "decode_parts.hpp"
#include "persist.hpp"

#include "../../include/flashrt_moe.h"

#include <map>
#include <mutex>
#include <set>
#include <tuple>
#include <utility>

namespace frt {

namespace {

constexpr int kNTW = kNTP;          // threads per workgroup
constexpr int kNWW = kNTW / 64;     // waves per workgroup
// The kernel is written for windows of up to 8 tokens (the reference's kMaxWindow; entries of at most
// 4 tokens, k_win_route's split) and takes those of 2-4 tokens. Measured on configs[1]-like windows (same box, the four-launch path
// beside it): T = 2 26.2 -> 23.5 us, T = 3 29.1 -> 25.8; but T = 5 35.9 -> 37.0 and T = 8 46.4 -> 47.7
// (at T = 8 each workgroup runs about 5 gate/up units one after another, where the four-launch
// path spreads them over 3 workgroups of 4 waves per CU), so larger windows keep the four launches.
constexpr int kWUseT = 4;
constexpr int kWLgStride = 4;       // words between two published logits (as k_dec1)
// logit and h words per thread to wait for, for windows of at most MT tokens: T (E + 1) logits,
// T (K + 1) ff / 32 9 h words
template <int MT>
struct DecwWait {
    static constexpr int lg = (MT * 1025 + kNTW - 1) / kNTW;
    static constexpr int h = MT <= 4 ? 16 : 25;
};

struct DecwArgs {
    const float* W;          // [E][n] router
    const float* bias;       // [E] or null
    const float* gate_w;     // [n] shared-expert gate
    const uint8_t* arena;    // routed expert 0
    const uint8_t* shared;
    size_t stride;
    const float* x;          // [T][n]
    const float* resid;      // [T][n] or null
    float* out;              // [T][n]
    float* logits;           // [T][E] plain copies of the logits (routing records), or null
    float* gate;             // [T] the shared gate logits, or null
    int32_t* ids;            // [T][K] rank order, or null
    float* wts;              // [T][K], or null
    uint32_t* counts;        // [E] or null
    Dec1Sync* sync;
    uint64_t* lg;            // [T][E + 1] tagged logits, kWLgStride words apart
    uint64_t* hb;            // [T (K + 1)][ff / 32][9] tagged h blocks of each compact slot (after the logits)
    uint64_t ticks;
    uint32_t* host_err;
    uint64_t* stamps;        // measurement only (null: none): [phase][workgroup] constant-clock ticks
    int T, E, K, ff, norm;
};
constexpr int kWPhases = 10;

typedef const __attribute__((address_space(4))) DecwArgs KWArgs;

template <int MT, int PASSES>
struct DecwLds {
    float cand_v[MT][128];
    int cand_id[MT][128];
    int32_t ids[MT][32];
    float w[MT][32];
    int rk[MT][32];           // rank of selection k by expert id
    uint32_t mask[1025];      // per expert (and E: the shared one), the tokens that chose it
    int ent_of[1025][2];      // per expert, its entries (tokens 0-3 and 4-7 of its list)
    int wtot[2][2];
    int comb_c[MT][33];       // token t's slots: routed in ascending expert id, then the shared one
    float comb_w[MT][33];
    float s_h[kDecMaxT][32];
    DecEntry ent[128];        // at most T (K + 1) <= 128 items
    int n_ent;
    __align__(16) float seq[kNWW][PASSES * 128];   // per wave: the gate/up block terms of seq_row_sums
};

// MT: the largest window of the instance (4, or 8 where the LDS allows)
template <int NB, int V, int NBF, int MT>
__global__ void __launch_bounds__(kNTW) k_decw(DecwArgs a_byval) {
    (void)a_byval;   // read where it lies (the kernel argument segment), as k_dec1 does
    const KWArgs& a = *(const KWArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int n = 64 * NB, L = NB;
    // dynamic: the inputs xs [T][64 (L + 1)] (each token's x by chain, chains padded by one float)
    // until they are quantized, then sh_q [NS][ff] | sh_d [NS][ff/32] | sh_y [NS][8]
    extern __shared__ __align__(16) uint8_t smem[];
    float* const xs0 = reinterpret_cast<float*>(smem);
    constexpr int XS = 64 * (L + 1);   // floats per token in xs
    __shared__ __align__(16) int8_t xq[MT][n];
    __shared__ float xd[MT][n / kQ8];
    __shared__ __align__(16) float s_lg[MT][64 * V + 4];
    __shared__ DecwLds<MT, gu_passes<NB, kNWW>()> S;
    __shared__ uint32_t s_ep[kNWW];
    __shared__ float s_r[MT];
    __shared__ uint64_t s_stamp[kWPhases];   // (kept in LDS, written out at the end)
#define FRT_DW_STAMP(ph)                                              \
    do {                                                              \
        if (a.stamps && threadIdx.x == 0) s_stamp[ph] = wall_clock64(); \
    } while (0)
    FRT_DW_STAMP(0);

    const int b = blockIdx.x, G = gridDim.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int T = a.T, E = a.E, K = a.K, ff = a.ff, K1 = K + 1, RB = ff / 32;
    const uint64_t deadline = wall_clock64() + a.ticks;
    {   // the epoch: the largest cell + 1 (k_dec1's rule; the cells are shared with it)
        uint32_t c = tid < G ? __hip_atomic_load(&a.sync->epoch[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        if (G > kNTW)
            for (int i = tid + kNTW; i < G; i += kNTW)
                c = max(c, __hip_atomic_load(&a.sync->epoch[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        for (int o = 32; o > 0; o >>= 1) c = max(c, uint32_t(__shfl_xor(int(c), o, 64)));
        if (lane == 0) s_ep[wave] = c;
    }

    // ---- 1. router rows (slot s = b + G w for wave w; slot E is the shared gate row), then the inputs
    const int s0 = b + wave * G;
    const bool rs = s0 <= E;
    float wr[L];
    if (rs) {
        const float* wrow = s0 < E ? a.W + size_t(s0) * n : a.gate_w;
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
    const float bias_v = (a.bias && rs && s0 < E) ? a.bias[s0] : 0.0f;
    {
        const float4* x4 = reinterpret_cast<const float4*>(a.x);
        for (int i = tid; i < T * (n / 4); i += kNTW) {
            const int t = i / (n / 4), e = 4 * (i % (n / 4));   // L % 4 == 0: a float4 stays within one chain
            const float4 v = x4[i];
            float* d = xs0 + t * XS + (e / L) * (L + 1) + e % L;
            d[0] = v.x;
            d[1] = v.y;
            d[2] = v.z;
            d[3] = v.w;
        }
    }
    __syncthreads();
    uint32_t ep = s_ep[0];
#pragma unroll
    for (int w = 1; w < kNWW; ++w) ep = max(ep, s_ep[w]);
    ep += 1u;
    const uint64_t err_val = (uint64_t(kErrMagic) << 32) | ep;
    const uint32_t tag = sync_tag(ep * uint32_t(kMaxStack));
    FRT_DW_STAMP(1);
    if (wave < T) {   // token `wave`'s RMS scale (LDS: the token index below is a runtime value)
        const float rt = a.norm ? rms_scale_wave<L>(xs0 + wave * XS + lane * (L + 1), n) : 1.0f;
        if (lane == 0) s_r[wave] = rt;
    }
    __syncthreads();
    auto router_dot = [&](int s, const float (&w)[L], float bv) {
        for (int t = 0; t < T; ++t) {
            const float* xc = xs0 + t * XS + lane * (L + 1);
            float acc = 0.0f;
            if (a.norm) {
#pragma unroll
                for (int i = 0; i < L; ++i) {
                    const float u = xc[i] * s_r[t];
                    acc = fmaf(w[i], u, acc);
                }
            } else {
#pragma unroll
                for (int i = 0; i < L; ++i) acc = fmaf(w[i], xc[i], acc);
            }
            acc = wave_sum_tree(acc);
            if (s < E && a.bias) acc = acc + bv;
            if (lane == 0) {
                pub(a.lg + (size_t(t) * (E + 1) + s) * kWLgStride, tag, __float_as_uint(acc));
                if (s < E) {
                    if (a.logits) a.logits[size_t(t) * E + s] = acc;
                } else if (a.gate) {
                    a.gate[t] = acc;
                }
            }
        }
    };
    if (rs) router_dot(s0, wr, bias_v);
    for (int s = s0 + kNWW * G; s <= E; s += kNWW * G) {   // only with fewer than (E + 1) / 8 workgroups
        float w2[L];
        const float* wrow = s < E ? a.W + size_t(s) * n : a.gate_w;
#pragma unroll
        for (int i = 0; i < L; ++i) w2[i] = wrow[lane * L + i];
        router_dot(s, w2, a.bias && s < E ? a.bias[s] : 0.0f);
    }
    FRT_DW_STAMP(2);
    if (wave >= kNWW / 2) {   // Q8_0 of the T inputs (u = x r with the norm) by the last 4 waves (with one
        // workgroup per CU they hold no router row below E = 4 G), while the first 4 compute theirs: a
        // lane pair per 32-block, 16 values a lane; T n / 32 is a multiple of 32, so every lane of a
        // wave runs the same number of rounds
        const int h = lane & 1, nblk = T * (n / kQ8);
        for (int p0 = (tid - kNTW / 2) >> 1; p0 < nblk; p0 += kNTW / 4) {
            const int t = p0 / (n / kQ8), blk = p0 % (n / kQ8);
            float v[16];
            float am = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int k = blk * kQ8 + 16 * h + j;
                v[j] = xs0[t * XS + (k / L) * (L + 1) + k % L];
                if (a.norm) v[j] = v[j] * s_r[t];
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
            uint32_t* dst = reinterpret_cast<uint32_t*>(&xq[t][blk * kQ8 + 16 * h]);
#pragma unroll
            for (int w = 0; w < 4; ++w) dst[w] = wq[w];
            if (h == 0) xd[t][blk] = f16_round(d);
        }
    }

    FRT_DW_STAMP(3);
    // ---- 2. all logits, the routing of each token, the entries, gate/up
    wait_words_at<DecwWait<MT>::lg, kNTW>([&](int i) { return a.lg + size_t(i) * kWLgStride; }, T * (E + 1), tag, deadline,
                                  &a.sync->err, err_val, a.host_err, [&](int i, uint32_t p) {
                                      const int t = i / (E + 1), e = i % (E + 1);
                                      s_lg[t][e] = __uint_as_float(p);
                                  });
    FRT_DW_STAMP(4);
    for (int e = tid; e <= E; e += kNTW) S.mask[e] = e == E ? (1u << T) - 1u : 0u;
    __syncthreads();
    if (wave < T) {   // token `wave`: ids and weights in rank order
        const int id = topk_wave_fast<V>(s_lg[wave], E, K, S.ids[wave], S.w[wave], S.cand_v[wave], S.cand_id[wave]);
        int rk = 0;   // the selection's rank by expert id among the token's (the ids are distinct)
        for (int k2 = 0; k2 < K; ++k2) rk += int(__builtin_amdgcn_readlane(id, k2) < id);
        if (lane < K) {
            S.rk[wave][lane] = rk;
            atomicOr(&S.mask[id], 1u << wave);
            if (b == 0) {   // the routing records, once
                if (a.ids) a.ids[wave * K + lane] = id;
                if (a.wts) a.wts[wave * K + lane] = S.w[wave][lane];
                if (a.counts) atomicAdd(a.counts + id, 1u);
            }
        }
    }
    __syncthreads();
    // the items i = t (K + 1) + k (k = K: the shared expert) in one entry per distinct expert, opened by
    // its first item, in order of first appearance (k_win_route's grouping; N = T (K + 1) <= 128: waves 0, 1)
    const int N = T * K1;
    const bool live = tid < N;
    const int it = tid / K1, ik = tid % K1;
    const int key = live ? (ik < K ? S.ids[it][ik] : E) : 0;
    const uint32_t m = live ? S.mask[key] : 0u;
    const int j = __popc(m & ((1u << it) - 1u)), tot = __popc(m);
    const bool opens = live && j % kDecMaxT == 0;   // an entry holds at most 4 tokens (k_win_route's split)
    const int nt = opens ? min(kDecMaxT, tot - j) : 0;
    int tu = 0, tb = 0;
    const int su = wave_excl_scan(int(opens), &tu), sb = wave_excl_scan(nt, &tb);
    if (lane == 0 && wave < 2) {
        S.wtot[0][wave] = tu;
        S.wtot[1][wave] = tb;
    }
    __syncthreads();
    if (opens) {
        const int u = (wave == 1 ? S.wtot[0][0] : 0) + su;
        DecEntry& d = S.ent[u];
        d.blob = key < E ? a.arena + size_t(key) * a.stride : a.shared;
        d.ntok = nt;
        d.base = (wave == 1 ? S.wtot[1][0] : 0) + sb;
        for (int q = 0; q < kDecMaxT; ++q) {
            d.tok[q] = 0;
            d.slot[q] = -1;
            d.w[q] = 0.0f;
        }
        S.ent_of[key][j / kDecMaxT] = u;
    }
    if (tid == 0) S.n_ent = S.wtot[0][0] + (N > 64 ? S.wtot[0][1] : 0);
    __syncthreads();
    if (live) {
        DecEntry& d = S.ent[S.ent_of[key][j / kDecMaxT]];
        const int sl = j % kDecMaxT;
        d.tok[sl] = it;
        d.slot[sl] = ik;
        d.w[sl] = 1.0f;
        const int c = d.base + sl;
        if (ik < K) {
            const int rk = S.rk[it][ik];
            S.comb_c[it][rk] = c;
            S.comb_w[it][rk] = S.w[it][ik];
        } else {
            S.comb_c[it][K] = c;
            S.comb_w[it][K] = sigmoidf_(s_lg[it][E]);
        }
    }
    __syncthreads();
    const int n_ent = S.n_ent, NU = n_ent * RB;
    FRT_DW_STAMP(5);

    // gate/up unit q: entry q / RB, ff rows 32 (q % RB) .. + 31, 32 / kNWW rows per wave
    constexpr int RPW = gu_rpw<NB>();   // rows per wave pass
    constexpr int ROWS = 32 / kNWW;
    constexpr int PASSES = gu_passes<NB, kNWW>();
    const int rsub = lane / NB, bk = lane % NB;
    const bool rlive = rsub < RPW;
    const int bl = rlive ? bk : 0;
    const size_t mb = mat_bytes(ff, n);
    struct GuRegs {
        uint4 cg[PASSES], cu[PASSES];
        uint32_t sg[PASSES], su[PASSES];
        uint32_t okm;
    };
    auto gu_load = [&](int q, GuRegs& g) {
        const DecEntry& e = S.ent[q / RB];
        const int rb = q % RB;
        const uint8_t* gcodes = e.blob;
        const uint16_t* gscal = reinterpret_cast<const uint16_t*>(e.blob + size_t(ff) * NB * 16);
        const uint8_t* ucodes = e.blob + mb;
        const uint16_t* uscal = reinterpret_cast<const uint16_t*>(e.blob + mb + size_t(ff) * NB * 16);
        g.okm = 0;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int rl = p * RPW + rsub;
            if (rlive && rl < ROWS) g.okm |= 1u << p;
            const int row = rb * 32 + wave * ROWS + min(rl, ROWS - 1);
            g.cg[p] = gld_u4_nt(gcodes + (size_t(row) * NB + bl) * 16);
            g.cu[p] = gld_u4_nt(ucodes + (size_t(row) * NB + bl) * 16);
            g.sg[p] = gld<uint16_t>(gscal + size_t(row) * NB + bl);
            g.su[p] = gld<uint16_t>(uscal + size_t(row) * NB + bl);
        }
    };
    auto gu_compute = [&](int q, const GuRegs& g) {
        const DecEntry& e = S.ent[q / RB];
        const int rb = q % RB;
        const int ntok = e.ntok;
        for (int jt = 0; jt < ntok; ++jt) {
            const int t = e.tok[jt];
            int xa[16];
            const int4* xp = reinterpret_cast<const int4*>(&xq[t][bl * kBlock]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int4 v = xp[k];
                xa[4 * k] = v.x;
                xa[4 * k + 1] = v.y;
                xa[4 * k + 2] = v.z;
                xa[4 * k + 3] = v.w;
            }
            const float xd0 = xd[t][2 * bl], xd1 = xd[t][2 * bl + 1];
            int xs0 = 0, xs1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) xs0 = dot4(xa[i], 0x01010101, xs0);
#pragma unroll
            for (int i = 8; i < 16; ++i) xs1 = dot4(xa[i], 0x01010101, xs1);
            float tg[PASSES], tu[PASSES];
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const uint32_t wg[4] = {g.cg[p].x, g.cg[p].y, g.cg[p].z, g.cg[p].w};
                const uint32_t wu[4] = {g.cu[p].x, g.cu[p].y, g.cu[p].z, g.cu[p].w};
                const bool okp = (g.okm >> p) & 1u;
                const float dg = okp ? h2f(uint16_t(g.sg[p])) : 0.0f, du = okp ? h2f(uint16_t(g.su[p])) : 0.0f;
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
            // the rows' sums in the CPU path's order (lane 2 RPW p + r: row p RPW + r)
            const float2 gu = seq_row_sums<NB, RPW, PASSES>(tg, tu, S.seq[wave], lane);
            const int p = lane / (2 * RPW), r = lane % (2 * RPW), row = p * RPW + r;
            if (r < RPW && p < PASSES && row < ROWS) S.s_h[jt][wave * ROWS + row] = gu.x / (1.0f + expf(-gu.x)) * gu.y;
        }
        __syncthreads();
        if (wave < ntok) {   // Q8_0 of token `wave`'s 32-row h block, published as 8 words of 4 codes and the scale
            const float v = lane < 32 ? S.s_h[wave][lane] : 0.0f;
            const float am = half_max(fabsf(v));
            const float d = q8_scale(am);
            const int c = q8_code(v, q8_inv(d)) & 0xff;
            const int l4 = (4 * lane) & 63;
            const uint32_t word = uint32_t(__shfl(c, l4)) | (uint32_t(__shfl(c, l4 + 1)) << 8) |
                                  (uint32_t(__shfl(c, l4 + 2)) << 16) | (uint32_t(__shfl(c, l4 + 3)) << 24);
            uint64_t* dst = a.hb + (size_t(e.base + wave) * RB + rb) * 9;
            if (lane < 8) pub(dst + lane, tag, word);
            if (lane == 8) pub(dst + 8, tag, __float_as_uint(f16_round(d)));
        }
        __syncthreads();   // s_h is free for the next unit
    };
    // a window has more units than workgroups (about 21 entries x ff / 32 at configs[1], 5 units per
    // workgroup at T = 8): two register sets in turn, unit i + 1's rows in flight while unit i computes
    {
        GuRegs g0, g1;
        if (b < NU) gu_load(b, g0);
        for (int q = b; q < NU; q += 2 * G) {
            if (q + G < NU) gu_load(q + G, g1);
            gu_compute(q, g0);
            if (q + G >= NU) break;
            if (q + 2 * G < NU) gu_load(q + 2 * G, g0);
            gu_compute(q + G, g1);
        }
    }

    FRT_DW_STAMP(6);
    // ---- 3. all h blocks, then the down rows and each token's combine
    const int NS = N;   // compact slots: one per item
    int8_t* sh_q = reinterpret_cast<int8_t*>(smem);
    float* sh_d = reinterpret_cast<float*>(smem + size_t(NS) * ff);
    float* sh_y = sh_d + size_t(NS) * (ff / kQ8);
    constexpr int BATCH = 3;   // entries per wave in the first (prefetched) batch: 24 entries
    const int r0 = 8 * b;
    const bool has_down = r0 < n;
    DownRegs<NBF, BATCH> D;
    if (has_down) down_load<NBF, BATCH, kNWW, true>(S.ent, n_ent, wave, r0, n, ff, D);   // land during the wait
    wait_words_at<DecwWait<MT>::h, kNTW>([&](int i) { return a.hb + i; }, NS * RB * 9, tag, deadline, &a.sync->err, err_val,
                                 a.host_err, [&](int i, uint32_t p) {
                                     const int c = i / (RB * 9), rem = i % (RB * 9), rb = rem / 9, part = rem % 9;
                                     if (part < 8) *reinterpret_cast<uint32_t*>(sh_q + size_t(c) * ff + rb * 32 + 4 * part) = p;
                                     else sh_d[c * (ff / kQ8) + rb] = __uint_as_float(p);
                                 });
    FRT_DW_STAMP(7);
    __syncthreads();
    auto combine = [&](int g0) {
        if (tid < 8 * T) {
            const int t = tid >> 3, rl = tid & 7, row = g0 + rl;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float p = S.comb_w[t][k] * sh_y[S.comb_c[t][k] * 8 + rl];
                acc = acc + p;
            }
            float o = acc + sh_y[S.comb_c[t][K] * 8 + rl] * S.comb_w[t][K];
            if (a.resid) o = a.resid[size_t(t) * n + row] + o;
            a.out[size_t(t) * n + row] = o;
        }
    };
    if (has_down) {
        down_compute<NBF, BATCH, kNWW>(S.ent, n_ent, wave, D, sh_q, sh_d, sh_y, ff);
        for (int u0 = wave + kNWW * BATCH; u0 < n_ent; u0 += kNWW * BATCH) {
            DownRegs<NBF, BATCH> D2;
            down_load<NBF, BATCH, kNWW, true>(S.ent, n_ent, u0, r0, n, ff, D2);
            down_compute<NBF, BATCH, kNWW>(S.ent, n_ent, u0, D2, sh_q, sh_d, sh_y, ff);
        }
        __syncthreads();
        FRT_DW_STAMP(8);
        combine(r0);
    }
    for (int g0 = r0 + 8 * G; g0 < n; g0 += 8 * G) {   // more 8-row groups than workgroups
        __syncthreads();   // sh_y of the previous group is combined
        for (int u0 = wave; u0 < n_ent; u0 += kNWW * BATCH) {
            DownRegs<NBF, BATCH> D2;
            down_load<NBF, BATCH, kNWW, true>(S.ent, n_ent, u0, g0, n, ff, D2);
            down_compute<NBF, BATCH, kNWW>(S.ent, n_ent, u0, D2, sh_q, sh_d, sh_y, ff);
        }
        __syncthreads();
        combine(g0);
    }
    FRT_DW_STAMP(9);
    if (a.stamps && tid == 0)
        for (int ph = 0; ph < kWPhases; ++ph) a.stamps[size_t(ph) * G + b] = s_stamp[ph];
#undef FRT_DW_STAMP
    if (tid == 0) __hip_atomic_store(&a.sync->epoch[b], ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_decw_zero(uint64_t* p, size_t words) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < words; i += size_t(gridDim.x) * blockDim.x) p[i] = 0;
}

std::mutex g_decw_mu;
std::set<std::pair<int, const void*>> g_decw_init;   // (device, sync region) already zeroed
std::map<std::tuple<int, const void*, size_t>, int> g_decw_grid;   // (device, kernel, LDS) -> grid size

}  // namespace

extern int g_dec1_grid_cap;
extern uint64_t g_dec1_ticks;
extern uint64_t* g_dec2_stamps;
size_t dec1_sync_bytes();
int dec1_eligible(int E, int K, int n, int ff);
int g_decw_on = 1;   // 1: windows of 2-4 tokens take this kernel where it fits (else the window path)

// the sync region's words of a call: T (E + 1) logits kWLgStride words apart, then the h blocks
static size_t decw_lg_bytes(int T, int E) { return up256(size_t(T) * (E + 1) * kWLgStride * 8); }
static size_t decw_sync_need(int T, int E, int K, int ff) {
    return kSyncHead + decw_lg_bytes(T, E) + size_t(T) * (K + 1) * (ff / 32) * 9 * 8;
}

// the dynamic LDS: the inputs by chain, later the h codes, scales and down rows of the NS slots
static size_t decw_smem(int T, int K, int n, int ff) {
    const size_t NS = size_t(T) * (K + 1);
    const size_t xs = size_t(T) * 64 * (n / 64 + 1) * 4, sh = NS * ff + NS * (ff / kQ8) * 4 + NS * 8 * 4;
    return xs > sh ? xs : sh;
}

template <typename Kern>
static int decw_go(Kern kern, DecwArgs& a, size_t smem, hipStream_t stream, bool probe_only) {
    int dev = 0;
    FRT_HIP(hipGetDevice(&dev));
    const void* kfn = reinterpret_cast<const void*>(kern);
    int grid;
    {
        std::lock_guard<std::mutex> lk(g_decw_mu);
        auto it = g_decw_grid.find({dev, kfn, smem});
        if (it == g_decw_grid.end()) {
            // every workgroup must be resident at once: one per CU, the kernel must fit with this LDS,
            // and it must need no private (scratch) memory
            int cus = 0, per_cu = 0;
            hipFuncAttributes fa{};
            FRT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
            FRT_HIP(hipFuncGetAttributes(&fa, kfn));
            if (fa.sharedSizeBytes + smem <= 160 * 1024) {
                FRT_HIP(hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, int(160 * 1024 - fa.sharedSizeBytes)));
                FRT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kNTW, smem));
            }
            grid = (per_cu >= 1 && cus >= 1 && fa.localSizeBytes == 0) ? (cus < kMaxGrid ? cus : kMaxGrid) : 0;
            g_decw_grid[{dev, kfn, smem}] = grid;
        } else {
            grid = it->second;
        }
    }
    if (grid < 1) return 1;
    if (g_dec1_grid_cap > 0 && g_dec1_grid_cap < grid) grid = g_dec1_grid_cap;
    if (probe_only) return kOk;
    launch_timed("decw_layer", kern, dim3(grid), dim3(kNTW), smem, stream, a);
    FRT_LAUNCHED("decode window");
    return kOk;
}

static int decw_run(DecwArgs& a, int n, size_t smem, hipStream_t stream, bool probe_only) {
    const int nb = n / 64, nbf = a.ff / 64;
    const bool v8 = a.E <= 512;
#define FRT_DWS(NBV, VV, NBFV) return decw_go(k_decw<NBV, VV, NBFV, kWUseT>, a, smem, stream, probe_only);
#define FRT_DWF(NBV, VV)              \
    switch (nbf) {                    \
        case 4: FRT_DWS(NBV, VV, 4)   \
        case 8: FRT_DWS(NBV, VV, 8)   \
        case 10: FRT_DWS(NBV, VV, 10) \
        case 16: FRT_DWS(NBV, VV, 16) \
    }                                 \
    break;
#define FRT_DWN(NBV)         \
    case NBV:                \
        if (v8) {            \
            FRT_DWF(NBV, 8)  \
        } else {             \
            FRT_DWF(NBV, 16) \
        }                    \
        break;
    switch (nb) {
        FRT_DWN(16) FRT_DWN(32) FRT_DWN(40) FRT_DWN(48) FRT_DWN(64)
    }
#undef FRT_DWN
#undef FRT_DWF
#undef FRT_DWS
    return set_error(kErrShape, "decode window: n=%d ff=%d", n, a.ff);
}

// Whether a window of T tokens can take this kernel (shape, the h words one wait covers, every
// workgroup resident with its LDS).
bool decw_support(int T, int E, int K, int n, int ff) {
    if (!g_decw_on || T < 2 || T > kWUseT || T * (K + 1) > 128 || !dec1_eligible(E, K, n, ff)) return false;
    const int hw = DecwWait<kWUseT>::h;
    if (size_t(T) * (K + 1) * (ff / 32) * 9 > size_t(hw) * kNTW) return false;
    if (decw_sync_need(T, E, K, ff) > dec1_sync_bytes()) return false;   // (the layer workspace's sync region)
    DecwArgs a{};
    a.T = T;
    a.E = E;
    a.K = K;
    a.ff = ff;
    return decw_run(a, n, decw_smem(T, K, n, ff), nullptr, true) == kOk;
}

int decw_layer(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared, int n, int ff, int norm, const float* resid,
               float* out, float* logits, float* gate, int32_t* ids, float* wts, uint32_t* counts, void* sync_ws,
               hipStream_t stream) {
    DecwArgs a{};
    a.W = W;
    a.bias = bias;
    a.gate_w = gate_w;
    a.arena = arena;
    a.shared = shared;
    a.stride = stride;
    a.x = x;
    a.resid = resid;
    a.out = out;
    a.logits = logits;
    a.gate = gate;
    a.ids = ids;
    a.wts = wts;
    a.counts = counts;
    a.T = T;
    a.E = E;
    a.K = K;
    a.ff = ff;
    a.norm = norm;
    int dev = 0;
    FRT_HIP(hipGetDevice(&dev));
    uint8_t* base = static_cast<uint8_t*>(sync_ws);
    a.sync = reinterpret_cast<Dec1Sync*>(base);
    a.lg = reinterpret_cast<uint64_t*>(base + kSyncHead);
    a.hb = reinterpret_cast<uint64_t*>(base + kSyncHead + decw_lg_bytes(T, E));   // (after this call's logits)
    a.ticks = g_dec1_ticks;
    a.stamps = g_dec2_stamps;
    if (int rc = host_err_flag(dev, !g_dec1_no_alloc, &a.host_err)) return rc;
    {
        std::lock_guard<std::mutex> lk(g_decw_mu);
        if (g_decw_init.insert({dev, sync_ws}).second) {   // a region not seen before is zeroed first
            k_decw_zero<<<64, 256, 0, stream>>>(reinterpret_cast<uint64_t*>(base), dec1_sync_bytes() / 8);
            FRT_LAUNCHED("decode window zero");
        }
    }
    const int rc = decw_run(a, n, decw_smem(T, K, n, ff), stream, false);
    return rc == 1 ? set_error(kErrShape, "decode window: the persistent grid does not fit (T=%d K=%d ff=%d)", T, K, ff)
                   : rc;
}

}  // namespace frt
