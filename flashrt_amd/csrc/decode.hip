// Decode / verify-window MoE (T <= 4 tokens): memory-bound fused dequant-GEMVs.
//
// Work list: one entry per distinct expert of the window (each expert's weights are read once for
// every token that selected it, arch/qwen4exp/moe_fast.cu:195-355), in ascending expert id, the
// shared expert last. Entry c-slots (entry u, token j) are numbered compactly (base[u] + j).
//
//   k_dec_route_gateup  per (32 ff rows, entry): every workgroup routes the window itself (top-k
//                 of each token, topk.hpp), so routing costs no launch; then gate and up rows of
//                 every token of its entry, SwiGLU, and Q8_0 of that 32-row block of h
//                 (quant/q2_0/moe_cpu.cpp:43-61 phase A). A window (T > 1): four waves per token
//                 route, every workgroup builds the whole entry list in LDS, and workgroup (0, 0)
//                 publishes ids, weights, entries and combine lists. A single token: one wave
//                 routes (route1_wave), each workgroup writes only its own entry, and workgroup
//                 (0, y) publishes entry y, its id and, formed while its weight rows load, its
//                 weight (workgroup (0, 0) also the weights in rank order).
//   k_dec_gateup  the same body for moe_hits, entries from k_hits_group
//   k_dec_down    per 8 output rows: down rows of every entry, then the weighted sum per token in
//                 expert order plus shared * sigmoid(gate) (moe_cpu.cpp:63-80 phase B and
//                 moe_ref.cu:90-97; a single token's combine list is the entry list itself); or,
//                 for moe_hits, the per-slot outputs yh.
//
// Inner product per (row, 64-block, token): the 16 code bytes are read as 4 dwords; (code >> 2s)
// & 0x03030303 lines up with activation dword 4s + w (the planar layout), so 16 v_dot4_i32_i8
// give sum(q * a) for both 32-halves exactly; the -1 offset uses the halves' code sums.
#include "decode_parts.hpp"


namespace frt {

namespace {

// ---- grouping of a window's (token, slot) items into entries (moe_fast.cu:195-232): distinct keys
// (blob pointers, or expert ids) in order of first appearance. An entry holds at most kDecMaxT
// tokens: the occurrences of a key beyond its entry's four slots open another entry at their place
// in that order (a key met five times in the window is read twice, once per entry). Item i = t K + k;
// an item's occurrence index j among the live items of its key decides its entry (the one opened by
// the key's occurrence 4 floor(j / 4)) and its slot in it (j mod 4); entries follow the items that
// open them, so the list is what a serial pass over the items builds. One workgroup of at least
// kHitsMaxItems threads (thread i: item i); s_key [kHitsMaxItems] holds the keys, s_live the flags.
constexpr int kHitsMaxItems = 128;
constexpr int kGenMaxN = 16384;   // moe_hits rows of any other shape: n and ff at most these
constexpr int kGenMaxFF = 4096;
struct GroupLds {
    uint64_t key[kHitsMaxItems];
    int live[kHitsMaxItems], j[kHitsMaxItems], u[kHitsMaxItems];
    int wtot[2][kHitsMaxItems / 64];
};
template <class BlobOf>
__device__ __forceinline__ void group_items(GroupLds& G, int N, int K, BlobOf blob_of, DecEntry* __restrict__ ent,
                                            int32_t* __restrict__ n_ent) {
    const int i = int(threadIdx.x);
    const bool in = i < kHitsMaxItems;
    const bool live = in && i < N && G.live[i];
    const uint64_t key = in ? G.key[i] : 0;
    int j = 0, tot = 0;
    if (live)
        for (int q = 0; q < N; ++q) {
            const bool same = G.live[q] && G.key[q] == key;
            j += int(same && q < i);
            tot += int(same);
        }
    const bool opens = live && j % kDecMaxT == 0;
    const int nt = opens ? min(kDecMaxT, tot - j) : 0;
    // exclusive scans over the items in order: entry index and compact base of each opener
    const int wave = i >> 6;
    int tu = 0, tb = 0;
    const int su = wave_excl_scan(int(opens), &tu), sb = wave_excl_scan(nt, &tb);
    if (in && (i & 63) == 0) {
        G.wtot[0][wave] = tu;
        G.wtot[1][wave] = tb;
    }
    if (in) G.j[i] = live ? j : -1;
    __syncthreads();
    int u0 = 0, b0 = 0;
    for (int w = 0; w < wave && w < kHitsMaxItems / 64; ++w) {
        u0 += G.wtot[0][w];
        b0 += G.wtot[1][w];
    }
    if (in) G.u[i] = u0 + su;
    if (i == 0) {
        int U = 0;
        for (int w = 0; w < kHitsMaxItems / 64; ++w) U += G.wtot[0][w];
        *n_ent = U;
    }
    __syncthreads();
    if (!live) return;
    int opener = i;   // the item of this key with occurrence index 4 floor(j / 4)
    for (int q = 0; q <= i; ++q)
        if (G.j[q] == j - j % kDecMaxT && G.key[q] == key) {
            opener = q;
            break;
        }
    const int u = G.u[opener], sl = j % kDecMaxT, t = i / K, k = i % K;
    DecEntry& d = ent[u];
    if (opens) {
        d.blob = blob_of(key);
        d.ntok = nt;
        d.base = b0 + sb;
        for (int q = nt; q < kDecMaxT; ++q) {   // the unused slots
            d.tok[q] = 0;
            d.slot[q] = -1;
            d.w[q] = 0.0f;
        }
    }
    d.tok[sl] = t;
    d.slot[sl] = k;
    d.w[sl] = 1.0f;
}

// moe_hits: the keys are the blob pointers; items k >= hit_n[t] take no part; no shared expert.
__global__ void __launch_bounds__(kHitsMaxItems) k_hits_group(const uint8_t* const* __restrict__ hit_ptr,
                                                              const int32_t* __restrict__ hit_n, int K, int T,
                                                              DecEntry* __restrict__ ent, int32_t* __restrict__ n_ent) {
    __shared__ GroupLds G;
    const int i = int(threadIdx.x), N = T * K;
    const int t = i / K, k = i % K;
    const bool live = i < N && k < min(hit_n[min(t, T - 1)], K);
    G.key[i] = live ? reinterpret_cast<uint64_t>(hit_ptr[i]) : 0;
    G.live[i] = int(live);
    __syncthreads();
    group_items(G, N, K, [](uint64_t key) { return reinterpret_cast<const uint8_t*>(key); }, ent, n_ent);
}

// A verify window's routing and grouping in one workgroup: wave t < T routes token t (topk.hpp, the
// k_route_topk selection: ids and renormalised weights, and the counts), then the (token, slot)
// items, the K routed experts of each token and the shared expert as slot K, are grouped into
// entries keyed by expert id (E: the shared expert), as group_items would: a token's ids are
// distinct, so an item's occurrence index is the number of earlier tokens that chose its expert,
// read off a per-expert mask of the tokens that chose it.
template <int V>
__global__ void __launch_bounds__(512) k_win_route(const float* __restrict__ logits, int T, int E, int K,
                                                   int32_t* __restrict__ ids, float* __restrict__ wts,
                                                   uint32_t* __restrict__ counts, const uint8_t* __restrict__ arena,
                                                   size_t stride, const uint8_t* __restrict__ shared_blob,
                                                   DecEntry* __restrict__ ent, int32_t* __restrict__ n_ent,
                                                   int32_t* __restrict__ arrive, int n_groups) {
    __shared__ float cand_v[8][128];
    __shared__ int cand_id[8][128];
    __shared__ int s_ids[8][32];
    __shared__ uint32_t s_mask[1025];   // per expert (and E: the shared one), the tokens that chose it
    __shared__ int s_ent[1025][2];      // per expert, its entries (tokens 0-3 and 4-7 of its list)
    __shared__ int s_wtot[2][2];
    const int wave = int(threadIdx.x) >> 6, lane = int(threadIdx.x) & 63, i = int(threadIdx.x);
    for (int e = i; e <= E; e += 512) s_mask[e] = e == E ? (1u << T) - 1u : 0u;
    for (int g = i; g < n_groups; g += 512)   // the down kernel's row-group counters
        __hip_atomic_store(arrive + g, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (wave < T) {
        const int id = topk_wave_fast<V>(logits + size_t(wave) * E, E, K, ids + size_t(wave) * K,
                                         wts + size_t(wave) * K, cand_v[wave], cand_id[wave]);
        if (lane < K) {
            s_ids[wave][lane] = id;
            atomicOr(&s_mask[id], 1u << wave);
            if (counts) atomicAdd(counts + id, 1u);
        }
    }
    __syncthreads();
    const int K1 = K + 1, N = T * K1;
    const bool live = i < N;   // N <= kHitsMaxItems <= 128: waves 0 and 1
    const int t = i / K1, k = i % K1;
    const int key = live ? (k < K ? s_ids[t][k] : E) : 0;
    const uint32_t m = live ? s_mask[key] : 0u;
    const int j = __popc(m & ((1u << t) - 1u)), tot = __popc(m);
    const bool opens = live && j % kDecMaxT == 0;
    const int nt = opens ? min(kDecMaxT, tot - j) : 0;
    int tu = 0, tb = 0;
    const int su = wave_excl_scan(int(opens), &tu), sb = wave_excl_scan(nt, &tb);
    if (lane == 0 && wave < 2) {
        s_wtot[0][wave] = tu;
        s_wtot[1][wave] = tb;
    }
    __syncthreads();
    const int u0 = wave == 1 ? s_wtot[0][0] : 0, b0 = wave == 1 ? s_wtot[1][0] : 0;
    const int u = u0 + su;
    if (opens) s_ent[key][j / kDecMaxT] = u;
    if (i == 0) *n_ent = s_wtot[0][0] + (N > 64 ? s_wtot[0][1] : 0);
    __syncthreads();
    if (!live) return;
    DecEntry& d = ent[s_ent[key][j / kDecMaxT]];
    const int sl = j % kDecMaxT;
    if (opens) {
        d.blob = key < E ? arena + size_t(key) * stride : shared_blob;
        d.ntok = nt;
        d.base = b0 + sb;
        for (int q = nt; q < kDecMaxT; ++q) {   // the unused slots
            d.tok[q] = 0;
            d.slot[q] = -1;
            d.w[q] = 0.0f;
        }
    }
    d.tok[sl] = t;
    d.slot[sl] = k;
    d.w[sl] = 1.0f;
}

// ---- gate + up for 32 ff rows of one entry by NW waves (32 / NW rows each). NB = n / 64 blocks
// per row; RPW rows per wave pass (64 / NB when NB divides 64, else 1 with NB <= 64 lanes live).
// With a down matrix `warm` (the entry's), the workgroup also loads the down rows that the down
// kernel's workgroups on this XCD will read (down workgroup i runs on XCD i % 8, like this one on
// XCD (linear id) % 8), so that their loads find them in this XCD's L2 rather than in HBM.
// This lane's activation block (16 dwords of Q8_0 codes and the two block scales) for each token
// slot of an entry: lane (row rsub, block b) reads block b (block 0 for a lane past the rows); a
// token slot past ntok repeats token 0 (skipped where used).
template <int MT>
struct DecAct {
    int xa[MT][16];
    float xd0[MT], xd1[MT];
};
template <int NB, int MT>
__device__ __forceinline__ void load_act(const int32_t* tok, int ntok, const int8_t* __restrict__ xq,
                                         const float* __restrict__ xd, int n, DecAct<MT>& a) {
    constexpr int RPW = (64 % NB == 0) ? 64 / NB : 1;
    const int lane = threadIdx.x & 63;
    const int bl = lane / NB < RPW ? lane % NB : 0;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        const int tj = tok[j < ntok ? j : 0];
        const int4* src = reinterpret_cast<const int4*>(xq + size_t(tj) * n + bl * kBlock);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int4 v = src[q];
            a.xa[j][4 * q + 0] = v.x;
            a.xa[j][4 * q + 1] = v.y;
            a.xa[j][4 * q + 2] = v.z;
            a.xa[j][4 * q + 3] = v.w;
        }
        a.xd0[j] = xd[size_t(tj) * (n / kQ8) + 2 * bl];
        a.xd1[j] = xd[size_t(tj) * (n / kQ8) + 2 * bl + 1];
    }
}

// Work a caller of gateup_body runs while the weight rows are in flight (after their loads are
// issued, before the first wait for them): a single token's routing weights (single_weights).
struct AfterLoads {
    float* wts = nullptr;          // the weights in rank order (workgroup (0, 0))
    DecEntry* ent_w = nullptr;     // this workgroup's published entry, whose w[0] becomes its weight
    const float* lg = nullptr;     // the selected logits in rank order (LDS)
    const DecEntry* e = nullptr;   // this workgroup's entry (rank in slot[0]; shared: gate logit in w[0])
    int K = 0;
    bool shared = false;           // the entry is the shared expert's
};
// As topk_weight_sel: e = exp(l - max) with max the rank-0 logit, w = e / (the sum of e in rank order
// from 0); the shared expert's weight is sigmoid(gate). One wave (lane k: rank k).
__device__ __forceinline__ void single_weights(const AfterLoads& a) {
    const int lane = threadIdx.x & 63;
    if (a.shared) {
        if (lane == 0) a.ent_w->w[0] = sigmoidf_(a.e->w[0]);
        return;
    }
    const bool r = lane < a.K;
    const float l = r ? a.lg[lane] : 0.0f;
    const float mx = a.lg[0];
    const float e = r ? expf(l - mx) : 0.0f;
    float ws = 0.0f;
    for (int k = 0; k < a.K; ++k) ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), k));
    const float w = e / ws;
    if (r && a.wts) a.wts[lane] = w;
    if (lane == a.e->slot[0]) a.ent_w->w[0] = w;
}

template <int NB, int NW, int MT = kDecMaxT>
__device__ __forceinline__ void gateup_body(const DecEntry& e, int rb, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                            int n, int ff, int8_t* __restrict__ hq, float* __restrict__ hd, float (*hrow)[32],
                            const uint8_t* warm = nullptr, const DecAct<MT>* pre = nullptr,
                            AfterLoads after_loads = {}) {
    constexpr int RPW = gu_rpw<NB>();
    constexpr int ROWS = 32 / NW;                       // rows per wave
    constexpr int PASSES = gu_passes<NB, NW>();
    __shared__ __align__(16) float seqbuf[NW][MT * 128];   // per wave: the block terms of seq_row_sums
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rsub = lane / NB, b = lane % NB;
    const bool live = rsub < RPW;
    const int nb = NB;
    const size_t mb = mat_bytes(ff, n);
    const uint8_t* gcodes = e.blob;
    const uint16_t* gscal = reinterpret_cast<const uint16_t*>(e.blob + size_t(ff) * nb * 16);
    const uint8_t* ucodes = e.blob + mb;
    const uint16_t* uscal = reinterpret_cast<const uint16_t*>(e.blob + mb + size_t(ff) * nb * 16);
    // loads in the order they are waited for (waits count in issue order): this lane's activation
    // block for each token (16 dwords and the two scales), then every pass's weights, then the
    // cache warming, which nothing here waits for until the end
    // (unconditional, with clamped indices: a token slot past ntok repeats token 0 and is skipped
    // below; a lane or row that is not live gets scale 0, so its products are 0)
    const int bl = live ? b : 0;
    DecAct<MT> act;
    if (pre) act = *pre;
    else load_act<NB, MT>(e.tok, e.ntok, xq, xd, n, act);
    const int(&xa)[MT][16] = act.xa;
    const float(&xd0)[MT] = act.xd0;
    const float(&xd1)[MT] = act.xd1;
    uint4 cg[PASSES], cu[PASSES];
    uint32_t sg[PASSES], su[PASSES];   // fp16 scale bits, one per register (no packing waits)
    uint32_t okm = 0;                  // bit p: pass p's row is real
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int rl = p * RPW + rsub;
        if (live && rl < ROWS) okm |= 1u << p;
        const int r = rb * 32 + wave * ROWS + min(rl, ROWS - 1);
        cg[p] = gld_u4(gcodes + (size_t(r) * nb + bl) * 16);
        cu[p] = gld_u4(ucodes + (size_t(r) * nb + bl) * 16);
        sg[p] = gld<uint16_t>(gscal + size_t(r) * nb + bl);
        su[p] = gld<uint16_t>(uscal + size_t(r) * nb + bl);
    }
    // warming: this workgroup's share of the down rows of the workgroups i = x + 8 m of the down
    // kernel (x this XCD; the nrb / 8 row-block workgroups of this entry on it split the m); a
    // down workgroup's rows are 8 code rows (8 NBF 16-byte chunks) and their 8 scale rows
    constexpr int NBF_W = 8;   // down blocks per row the warming is laid out for (ff = 512)
    uint4 wv[2];
    const int nrb = ff / 32;   // row-block workgroups per entry (the grid's x extent; kept out of
                               // the dispatch packet, whose load would be waited for here)
    const bool do_warm = warm && ff == 64 * NBF_W && nrb % 8 == 0 && (n / 8) % 8 == 0;
    {   // unconditional (without warming: two harmless loads of this entry's first bytes)
        const int lin = rb + nrb * int(blockIdx.y);
        const int x = lin % 8, P = max(nrb / 8, 1), q = rb / 8;
        constexpr int CH = 8 * NBF_W + 8 * NBF_W * 2 / 16;   // 16-byte chunks per down workgroup: 64 + 8
        const int per = (n / 8 / 8 + P - 1) / P;              // down workgroups this one warms
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int c = min(int(threadIdx.x) + k * 64 * NW, per * CH - 1);
            const int i = min(x + 8 * (q + P * (c / CH)), n / 8 - 1), kk = c % CH;
            const size_t off = kk < 8 * NBF_W ? (size_t(i) * 8 * NBF_W + kk) * 16
                                              : size_t(n) * NBF_W * 16 + size_t(i) * 8 * NBF_W * 2 + (kk - 8 * NBF_W) * 16;
            wv[k] = gld_u4(do_warm ? warm + off : e.blob);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (after_loads.ent_w && (threadIdx.x >> 6) == 0) single_weights(after_loads);
    int xs0[MT], xs1[MT];   // the halves' code sums
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s0 = dot4(xa[j][i], 0x01010101, s0);
#pragma unroll
        for (int i = 8; i < 16; ++i) s1 = dot4(xa[j][i], 0x01010101, s1);
        xs0[j] = s0;
        xs1[j] = s1;
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const uint32_t wg[4] = {cg[p].x, cg[p].y, cg[p].z, cg[p].w};
        const uint32_t wu[4] = {cu[p].x, cu[p].y, cu[p].z, cu[p].w};
        const bool okp = (okm >> p) & 1u;
        const float dg = okp ? h2f(uint16_t(sg[p])) : 0.0f, du = okp ? h2f(uint16_t(su[p])) : 0.0f;
        float ag[MT], au[MT];
#pragma unroll
        for (int j = 0; j < MT; ++j) ag[j] = au[j] = 0.0f;
        // integer dots per token and half
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            if (j >= e.ntok) continue;
            int g0 = 0, g1 = 0, u0 = 0, u1 = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                g0 = dot4(int(wg[w] & 0x03030303u), xa[j][w], g0);
                g0 = dot4(int((wg[w] >> 2) & 0x03030303u), xa[j][4 + w], g0);
                g1 = dot4(int((wg[w] >> 4) & 0x03030303u), xa[j][8 + w], g1);
                g1 = dot4(int((wg[w] >> 6) & 0x03030303u), xa[j][12 + w], g1);
                u0 = dot4(int(wu[w] & 0x03030303u), xa[j][w], u0);
                u0 = dot4(int((wu[w] >> 2) & 0x03030303u), xa[j][4 + w], u0);
                u1 = dot4(int((wu[w] >> 4) & 0x03030303u), xa[j][8 + w], u1);
                u1 = dot4(int((wu[w] >> 6) & 0x03030303u), xa[j][12 + w], u1);
            }
            const float fg = float(g0 - xs0[j]) * xd0[j] + float(g1 - xs1[j]) * xd1[j];
            const float fu = float(u0 - xs0[j]) * xd0[j] + float(u1 - xs1[j]) * xd1[j];
            ag[j] = fg * dg;
            au[j] = fu * du;
        }
        // the rows' sums over their NB lanes in the CPU path's order: lane 2 RPW j + r holds token j's
        // row p RPW + r
        const float2 gu = seq_row_sums<NB, RPW, MT>(ag, au, seqbuf[wave], lane);
        const int j = lane / (2 * RPW), r = lane % (2 * RPW);
        if (j < e.ntok && r < RPW && p * RPW + r < ROWS)
            hrow[j][wave * ROWS + p * RPW + r] = gu.x / (1.0f + expf(-gu.x)) * gu.y;
    }
    __syncthreads();
    // Q8_0 of the 32-row block of h for each token: wave w < ntok, lanes 0..31
    if (wave < e.ntok) {   // the whole wave takes part in the DPP max; lanes 0..31 hold the block
        const float v = lane < 32 ? hrow[wave][lane] : 0.0f;
        const float am = half_max(fabsf(v));
        const float d = q8_scale(am);
        const float id = q8_inv(d);
        const int c = e.base + wave;
        if (lane < 32) hq[size_t(c) * ff + rb * 32 + lane] = int8_t(q8_code(v, id));
        if (lane == 0) hd[size_t(c) * (ff / kQ8) + rb] = f16_round(d);
    }
    if (do_warm && n < 0)   // keeps the warming loads (n > 0 always); every dword, so that no register of
                            // a load in flight is reused before it lands
        hd[0] = float(wv[0].x ^ wv[0].y ^ wv[0].z ^ wv[0].w ^ wv[1].x ^ wv[1].y ^ wv[1].z ^ wv[1].w);
}

// Four waves per workgroup (8 ff rows each): at n <= 2048 three workgroups fit per CU without
// register spills (12 waves, against 8 for one 8-wave workgroup); wider rows fit two.
template <int NB>
__global__ void __launch_bounds__(256, NB > 32 ? 2 : 3) k_dec_gateup(const DecEntry* __restrict__ ent, const int32_t* __restrict__ n_ent,
                                                    const int8_t* __restrict__ xq, const float* __restrict__ xd, int n,
                                                    int ff, int8_t* __restrict__ hq, float* __restrict__ hd) {
    __shared__ float hrow[kDecMaxT][32];
    if (int(blockIdx.y) >= *n_ent) return;
    const DecEntry e = ent[blockIdx.y];
    gateup_body<NB, 4>(e, blockIdx.x, xq, xd, n, ff, hq, hd, hrow);
}

template <int NB, int V, int MT>
__global__ void __launch_bounds__(1024) k_dec_route_gateup(const float* __restrict__ logits,
                                                          const float* __restrict__ gate, int T, int E, int K,
                                                          const uint8_t* __restrict__ arena, size_t stride,
                                                          const uint8_t* __restrict__ shared_blob,
                                                          const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                          int n, int ff, int8_t* __restrict__ hq,
                                                          float* __restrict__ hd, DecEntry* __restrict__ ent_out,
                                                          int32_t* __restrict__ n_ent_out, DecComb* __restrict__ comb_out,
                                                          int32_t* __restrict__ ids, float* __restrict__ wts,
                                                          uint32_t* counts) {
    __shared__ WinLds L;
    __shared__ float hrow[kDecMaxT][32];
    // a single token (MT = 1): its activation block does not depend on the routing, so its loads
    // are issued right behind the logits' and land during the routing
    DecAct<MT> pre;
    auto preload = [&]() {
        if (MT == 1) {
            const int32_t tok0[1] = {0};
            load_act<NB, MT>(tok0, 1, xq, xd, n, pre);
        }
    };
    const int U1 = window_entries<V>(logits, gate, T, E, K, arena, stride, shared_blob, L, preload);
    if (T == 1) {
        // a single token: workgroup (0, y) publishes entry y, the id of its selection (rank slot[0])
        // and its count; its weight (and workgroup (0, 0) the weights in rank order) it forms while
        // its weight rows load (single_weights)
        const int y = int(blockIdx.y);
        if (blockIdx.x == 0 && y < U1) {
            constexpr int kW0 = int(offsetof(DecEntry, w) / 4);   // w[0]: the weight, written later
            if (threadIdx.x < int(sizeof(DecEntry) / 4) && int(threadIdx.x) != kW0)
                reinterpret_cast<int32_t*>(ent_out + y)[threadIdx.x] = reinterpret_cast<const int32_t*>(&L.ent[y])[threadIdx.x];
            if (threadIdx.x == 0 && y < K) {
                const int id = L.ids[0][L.ent[y].slot[0]];
                ids[L.ent[y].slot[0]] = id;
                if (counts) atomicAdd(counts + id, 1u);
            }
            if (threadIdx.x == 0 && y == 0) *n_ent_out = U1;
        }
    } else if (blockIdx.x == 0 && blockIdx.y == 0) {
        for (int i = threadIdx.x; i < U1 * int(sizeof(DecEntry) / 4); i += blockDim.x)
            reinterpret_cast<int32_t*>(ent_out)[i] = reinterpret_cast<const int32_t*>(L.ent)[i];
        if (threadIdx.x < T * K) {
            const int t = threadIdx.x / K, k = threadIdx.x % K;
            ids[t * K + k] = L.ids[t][k];
            wts[t * K + k] = L.w[t][k];
            if (counts) atomicAdd(counts + L.ids[t][k], 1u);
        }
        for (int i = threadIdx.x; i < int(sizeof(DecComb) / 4); i += blockDim.x)
            reinterpret_cast<int32_t*>(comb_out)[i] = reinterpret_cast<const int32_t*>(&L.comb)[i];
        if (threadIdx.x == 0) *n_ent_out = U1;
    }
    if (int(blockIdx.y) >= U1) return;
    const DecEntry e = L.ent[blockIdx.y];
    AfterLoads al;
    if (T == 1 && blockIdx.x == 0) {
        al.wts = blockIdx.y == 0 ? wts : nullptr;
        al.ent_w = ent_out + blockIdx.y;
        al.lg = L.w[0];
        al.e = &L.ent[blockIdx.y];
        al.K = K;
        al.shared = int(blockIdx.y) == K;
    }
    gateup_body<NB, 16, MT>(e, blockIdx.x, xq, xd, n, ff, hq, hd, hrow, e.blob + 2 * mat_bytes(ff, n),
                            MT == 1 ? &pre : nullptr, al);
}

// combine of token t, down row rl (of the workgroup's 8) from its combine list: the K routed slots
// in ascending expert id, each weight * y summed from 0, then + the shared expert's y * sigmoid(gate)
// (moe_cpu.cpp:63-80 phase B order; moe_ref.cu:90-97). Every LDS read is issued before the sum.
__device__ __forceinline__ float combine_list(const DecComb& C, int K, int t, int rl, const float* sh_y) {
    constexpr int RD = 8;
    float wv[32], yv[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int kk = k < K ? k : 0;
        wv[k] = C.w[t][kk];
        yv[k] = sh_y[C.slot[t][kk] * RD + rl];
    }
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if (k < K) {
            const float p = wv[k] * yv[k];
            acc = acc + p;
        }
    const float p = sh_y[C.slot[t][K] * RD + rl] * C.w[t][K];
    return acc + p;
}

// ---- down for 8 output rows x every entry, then the combine. NBF = ff / 64 (8 lanes per row
// when ff = 512). 256 threads; wave w takes entries w, w + 4, ...
// ONE: a single token's layer (T = 1, no per-slot outputs): its combine list is the entry list itself
// (entry u = compact slot u, ascending expert id, the shared expert last, weight w[0]), so the list
// is not staged and the sum reads the entries.
template <int NBF, bool MAYBE_EMPTY, bool ONE>
__global__ void __launch_bounds__(256) k_dec_down(const DecEntry* ent_g, const int32_t* __restrict__ n_ent,
                                                  const DecComb* __restrict__ comb,
                                                  const int8_t* __restrict__ hq, const float* __restrict__ hd, int n,
                                                  int ff, int T, int K, const float* __restrict__ resid,
                                                  float* __restrict__ out, float* __restrict__ yh, int U_max,
                                                  int S_max, const float* __restrict__ pf, int pf_rows) {
    constexpr int RD = 8;   // rows per workgroup
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ DecEntry s_ent[kDecMaxEnt];
    __shared__ DecComb s_comb;
    // every global load is issued before the first wait: the residual this thread adds in the
    // combine, the entry count, the LDS staging of the entry list and the quantized hidden vectors,
    // and the first batch of down rows (their blob pointers read straight from the global entry list)
    const int r0 = blockIdx.x * RD;
    const int ti = threadIdx.x / RD, rli = threadIdx.x % RD;
    const float res = (resid && ti < T) ? resid[size_t(ti) * n + r0 + rli] : 0.0f;
    const int U = *n_ent;
    if (MAYBE_EMPTY && U == 0) return;   // moe_hits with no hits: nothing to write
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the staging loads go first: a wait for them (wait counts run in issue order) then does not
    // also wait for the down rows issued after them
    int8_t* sh_q = reinterpret_cast<int8_t*>(smem);                        // [S_max][ff]
    float* sh_d = reinterpret_cast<float*>(smem + size_t(S_max) * ff);    // [S_max][ff/32]
    float* sh_y = sh_d + size_t(S_max) * (ff / kQ8);                       // [S_max][RD]
    const int n_e = U_max * int(sizeof(DecEntry) / 16), n_c = int(sizeof(DecComb) / 4), n_q = S_max * ff / 16,
              n_d = S_max * (ff / kQ8);
    Stage<int4, 1, 256> st_e;
    Stage<int32_t, 2, 256> st_c;
    Stage<int4, 3, 256> st_q;
    Stage<float, 2, 256> st_d;
    st_e.load(reinterpret_cast<const int4*>(ent_g), n_e);
    if (!ONE) st_c.load(reinterpret_cast<const int32_t*>(comb), n_c);
    st_q.load(reinterpret_cast<const int4*>(hq), n_q);
    st_d.load(hd, n_d);
    DownRegs<NBF, 4> R;
    down_load<NBF, 4>(ent_g, U, wave, r0, n, ff, R);   // global entry list (down_load reads it as global)
    __builtin_amdgcn_sched_barrier(0);
    st_e.store(reinterpret_cast<int4*>(s_ent), reinterpret_cast<const int4*>(ent_g), n_e);
    if (!ONE && !yh) st_c.store(reinterpret_cast<int32_t*>(&s_comb), reinterpret_cast<const int32_t*>(comb), n_c);
    st_q.store(reinterpret_cast<int4*>(sh_q), reinterpret_cast<const int4*>(hq), n_q);
    st_d.store(sh_d, hd, n_d);
    __syncthreads();
    // cache warming, after every load this kernel waits for before its end (waits count in issue
    // order): rows 2 b, 2 b + 1 of the next layer's router, read there by router workgroup b on
    // this XCD
    float4 pv[4];
    const bool do_pf = pf && 2 * int(blockIdx.x) + 1 < pf_rows;
    if (do_pf) {
        const float4* src = reinterpret_cast<const float4*>(pf + size_t(2 * blockIdx.x) * n);
#pragma unroll
        for (int k = 0; k < 4; ++k) pv[k] = src[min(k * 256 + int(threadIdx.x), n / 2 - 1)];
    }
    const DecEntry* ent = s_ent;
    down_compute<NBF, 4>(ent, U, wave, R, sh_q, sh_d, sh_y, ff);
    for (int u0 = wave + 16; u0 < U; u0 += 16) {
        DownRegs<NBF, 4> R2;
        down_load<NBF, 4>(ent_g, U, u0, r0, n, ff, R2);
        down_compute<NBF, 4>(ent, U, u0, R2, sh_q, sh_d, sh_y, ff);
    }
    __syncthreads();
    if (yh) {   // moe_hits: per-slot outputs
        const int S = ent[U - 1].base + ent[U - 1].ntok;
        for (int i = threadIdx.x; i < S * RD; i += blockDim.x) {
            const int c = i / RD, rl = i % RD;
            int u = 0;
            while (ent[u].base + ent[u].ntok <= c) ++u;
            const int j = c - ent[u].base;
            yh[(size_t(ent[u].tok[j]) * K + ent[u].slot[j]) * n + r0 + rl] = sh_y[c * RD + rl];
        }
        return;
    }
    if (ti < T) {
        float o;
        if (ONE) {   // the combine_list order: the K routed entries from 0, then the shared one
            float acc = 0.0f;
            for (int u = 0; u < K; ++u) {
                const float p = ent[u].w[0] * sh_y[u * RD + rli];
                acc = acc + p;
            }
            o = acc + sh_y[K * RD + rli] * ent[K].w[0];
        } else {
            o = combine_list(s_comb, K, ti, rli, sh_y);
        }
        if (resid) o = res + o;
        out[size_t(ti) * n + r0 + rli] = o;
    }
    if (do_pf) {   // keeps the warming loads
        float z = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) z += pv[k].x + pv[k].y + pv[k].z + pv[k].w;
        if (n < 0) out[0] = z;   // n > 0 always
    }
}


// ---- moe_hits down with per-slot outputs: workgroup (x, y) takes output rows 8x .. 8x + 7 of entries
// 8y .. 8y + 7 (4 waves x 2 entries), staging only those entries' hidden vectors (their compact
// slots are contiguous); no sum across entries, so the entry chunks are independent workgroups.
// (Measured per window of T = 2 / 3 / 5 / 8 tokens: 8 entries per workgroup 1.2 / 1.5 / 1.3 / 3.2 us
// faster than 16; 4 entries 0.2 us faster at T <= 3, 1.6-2.0 us slower at T >= 5.)
constexpr int kHitsDownEnt = 8;
constexpr int kHitsBatch = kHitsDownEnt / 4;   // entries per wave
// A verify window's combine, fused into the down kernel: the last workgroup of a row group to
// finish (a counter per row group, zeroed by k_win_route) sums that group's rows for every token.
struct WinComb {
    int32_t* arrive;        // [n / 8]; null: no combine (moe_hits)
    const int32_t* ids;     // [T][K] rank order
    const float* wts;       // [T][K]
    const float* gate;      // [T] shared-expert gate logits
    const float* resid;     // [T][n] or null
    float* out;             // [T][n]
    int T, K;               // K routed slots per token (the shared expert is slot K)
};
template <int NBF>
__global__ void __launch_bounds__(256) k_hits_down(const DecEntry* __restrict__ ent_g, const int32_t* __restrict__ n_ent,
                                                   const int8_t* __restrict__ hq, const float* __restrict__ hd, int n,
                                                   int ff, int K, float* __restrict__ yh, WinComb wc) {
    constexpr int RD = 8;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ DecEntry s_ent[kHitsDownEnt];
    const int U = *n_ent, u_lo = int(blockIdx.y) * kHitsDownEnt;
    if (u_lo >= U) return;
    const int nu = min(U - u_lo, kHitsDownEnt);
    const int r0 = blockIdx.x * RD, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const DecEntry* eg = ent_g + u_lo;
    const int c_lo = eg[0].base, c_hi = eg[nu - 1].base + eg[nu - 1].ntok;   // this chunk's compact slots
    const int nc = c_hi - c_lo;
    int8_t* sh_q = reinterpret_cast<int8_t*>(smem);                       // [nc][ff]
    float* sh_d = reinterpret_cast<float*>(smem + size_t(kHitsDownEnt * kDecMaxT) * ff);   // [nc][ff/32]
    float* sh_y = sh_d + size_t(kHitsDownEnt * kDecMaxT) * (ff / kQ8);                     // [nc][RD]
    // staging loads first (waits count in issue order), then the down rows, then the LDS stores
    const int nq = nc * ff / 16, nd = nc * (ff / kQ8);
    const int4* srcq = reinterpret_cast<const int4*>(hq + size_t(c_lo) * ff);
    const float* srcd = hd + size_t(c_lo) * (ff / kQ8);
    int4 vq[4];
    float vd[2];
#pragma unroll
    for (int k = 0; k < 4; ++k) vq[k] = srcq[min(tid + 256 * k, nq - 1)];
#pragma unroll
    for (int k = 0; k < 2; ++k) vd[k] = srcd[min(tid + 256 * k, nd - 1)];
    DownRegs<NBF, kHitsBatch> R;
    down_load<NBF, kHitsBatch>(eg, nu, wave, r0, n, ff, R);
    __builtin_amdgcn_sched_barrier(0);
    if (tid < nu * int(sizeof(DecEntry) / 4))
        reinterpret_cast<int32_t*>(s_ent)[tid] = reinterpret_cast<const int32_t*>(eg)[tid];
    int4* dq = reinterpret_cast<int4*>(sh_q);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (tid + 256 * k < nq) dq[tid + 256 * k] = vq[k];
    for (int i = tid + 1024; i < nq; i += 256) dq[i] = srcq[i];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        if (tid + 256 * k < nd) sh_d[tid + 256 * k] = vd[k];
    for (int i = tid + 512; i < nd; i += 256) sh_d[i] = srcd[i];
    __syncthreads();
    // entries indexed locally, slots globally: the LDS arrays are offset by the chunk's first slot
    down_compute<NBF, kHitsBatch>(s_ent, nu, wave, R, sh_q - size_t(c_lo) * ff, sh_d - size_t(c_lo) * (ff / kQ8),
                         sh_y - size_t(c_lo) * RD, ff);
    __syncthreads();
    for (int i = tid; i < nc * RD; i += 256) {
        const int c = c_lo + i / RD, rl = i % RD;
        int u = 0;
        while (s_ent[u].base + s_ent[u].ntok <= c) ++u;
        const int j = c - s_ent[u].base;
        float* dst = yh + (size_t(s_ent[u].tok[j]) * K + s_ent[u].slot[j]) * n + r0 + rl;
        if (wc.arrive) __hip_atomic_store(dst, sh_y[(c - c_lo) * RD + rl], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else *dst = sh_y[(c - c_lo) * RD + rl];
    }
    if (!wc.arrive) return;
    // out[t] = resid[t] + (sum over the routed slots in ascending expert id of w * y, from 0) +
    // y_shared * sigmoid(gate[t]) (moe_cpu.cpp:63-80 phase B order; moe_ref.cu:90-97), by the row
    // group's last workgroup. The rows go out as agent-scope stores (to the memory side, past this
    // XCD's L2), each wave waits for their completion, and only then is the workgroup counted in;
    // the last one reads the rows with agent-scope loads. (A release / acquire fence pair would write
    // back and invalidate whole L2s, which costs the following kernels their cached weights.)
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's stores are complete
    __syncthreads();
    if (tid == 0) {
        const int ny = (U + kHitsDownEnt - 1) / kHitsDownEnt;
        s_last = __hip_atomic_fetch_add(wc.arrive + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ny - 1;
    }
    __syncthreads();
    if (!s_last) return;
    // (the staging area is free again: every wave has passed the barrier above)
    float(*s_yc)[33] = reinterpret_cast<float(*)[33]>(smem);   // [token, row][slot]
    int(*s_order)[32] = reinterpret_cast<int(*)[32]>(smem + sizeof(float) * kDecMaxHitsT * RD * 33);
    const int Kr = wc.K;
    // every slot row of the group at once (one memory round trip), parked in LDS
    for (int i = tid; i < wc.T * RD * (Kr + 1); i += 256) {
        const int tr = i % (wc.T * RD), k = i / (wc.T * RD), t = tr / RD;
        s_yc[tr][k] = __hip_atomic_load(yh + (size_t(t) * K + k) * n + r0 + tr % RD, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < wc.T * Kr) {   // rank of slot k by expert id (one token's ids are distinct)
        const int t = tid / Kr, k = tid % Kr, e = wc.ids[t * Kr + k];
        int r = 0;
        for (int q = 0; q < Kr; ++q) r += wc.ids[t * Kr + q] < e ? 1 : 0;
        s_order[t][r] = k;
    }
    __syncthreads();
    if (tid < wc.T * RD) {
        const int t = tid / RD, row = r0 + tid % RD;
        const float* yc = s_yc[tid];
        float acc = 0.0f;
        for (int r = 0; r < Kr; ++r) {
            const int k = s_order[t][r];
            const float p = wc.wts[t * Kr + k] * yc[k];
            acc = acc + p;
        }
        const float p = yc[Kr] * sigmoidf_(wc.gate[t]);
        float o = acc + p;
        if (wc.resid) o = wc.resid[size_t(t) * n + row] + o;
        wc.out[size_t(t) * n + row] = o;
    }
}

// ---- moe_hits at any shape of the reference's envelope (n a multiple of 512, ff a multiple of 64 up
// to 4096; arch/qwen4exp/moe_fast.cu:557): the same products with the row length a runtime value. Each
// lane walks the 64-blocks lane, lane + 64, ... of a row; the activation blocks are read from the
// global Q8_0 input (L1 / L2 hits after the first row). Float order: the block terms are added one
// after another, blocks ascending (the shapes of the templated kernels keep those kernels).
// Gate / up: workgroup (rb, u) takes ff rows 32 rb .. 32 rb + 31 of entry u, 8 rows per wave; SwiGLU
// and Q8_0 of the 32-row h block per token, as gateup_body.
__global__ void __launch_bounds__(256) k_gen_gateup(const DecEntry* __restrict__ ent, const int32_t* __restrict__ n_ent,
                                                    const int8_t* __restrict__ xq, const float* __restrict__ xd, int n,
                                                    int ff, int8_t* __restrict__ hq, float* __restrict__ hd) {
    __shared__ float hrow[kDecMaxT][32];
    __shared__ float terms[4][2 * kDecMaxT][kGenMaxN / kBlock];   // per wave: a row's block terms by token
    if (int(blockIdx.y) >= *n_ent) return;
    const DecEntry e = ent[blockIdx.y];
    const int rb = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nb = n / kBlock;
    const size_t mb = mat_bytes(ff, n);
    const uint8_t* gcodes = e.blob;
    const uint16_t* gscal = reinterpret_cast<const uint16_t*>(e.blob + size_t(ff) * nb * 16);
    const uint8_t* ucodes = e.blob + mb;
    const uint16_t* uscal = reinterpret_cast<const uint16_t*>(e.blob + mb + size_t(ff) * nb * 16);
    for (int i = 0; i < 8; ++i) {
        const int r = rb * 32 + wave * 8 + i;
        for (int b = lane; b < nb; b += 64) {
            const uint4 cg = gld_u4(gcodes + (size_t(r) * nb + b) * 16);
            const uint4 cu = gld_u4(ucodes + (size_t(r) * nb + b) * 16);
            const float dg = h2f(gld<uint16_t>(gscal + size_t(r) * nb + b));
            const float du = h2f(gld<uint16_t>(uscal + size_t(r) * nb + b));
            const uint32_t wg[4] = {cg.x, cg.y, cg.z, cg.w}, wu[4] = {cu.x, cu.y, cu.z, cu.w};
#pragma unroll
            for (int j = 0; j < kDecMaxT; ++j) {
                if (j >= e.ntok) break;
                const int t = e.tok[j];
                const int4* src = reinterpret_cast<const int4*>(xq + size_t(t) * n + size_t(b) * kBlock);
                int xa[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int4 v = src[q];
                    xa[4 * q] = v.x;
                    xa[4 * q + 1] = v.y;
                    xa[4 * q + 2] = v.z;
                    xa[4 * q + 3] = v.w;
                }
                int s0 = 0, s1 = 0, g0 = 0, g1 = 0, u0 = 0, u1 = 0;
#pragma unroll
                for (int q = 0; q < 8; ++q) s0 = dot4(xa[q], 0x01010101, s0);
#pragma unroll
                for (int q = 8; q < 16; ++q) s1 = dot4(xa[q], 0x01010101, s1);
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
                const float xd0 = xd[size_t(t) * (n / kQ8) + 2 * b], xd1 = xd[size_t(t) * (n / kQ8) + 2 * b + 1];
                const float fg = float(g0 - s0) * xd0 + float(g1 - s1) * xd1;
                const float fu = float(u0 - s0) * xd0 + float(u1 - s1) * xd1;
                terms[wave][2 * j][b] = fg * dg;
                terms[wave][2 * j + 1][b] = fu * du;
            }
        }
        // the row's sums in the CPU path's order (matvec_ref: blocks ascending from 0): lane 2 j adds
        // token j's gate terms, lane 2 j + 1 its up terms
        // the wave's LDS operations complete in order; the empty asm keeps the compiler from moving the
    // reads of other lanes' terms above the stores
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
        float sum = 0.0f;
        if (lane < 2 * e.ntok)
            for (int b = 0; b < nb; ++b) sum = sum + terms[wave][lane][b];
        asm volatile("" ::: "memory");   // the next row's stores stay after these reads
        __builtin_amdgcn_wave_barrier();
        const float up = __shfl(sum, min(lane + 1, 63));
        if (lane < 2 * e.ntok && (lane & 1) == 0) hrow[lane >> 1][wave * 8 + i] = sum / (1.0f + expf(-sum)) * up;
    }
    __syncthreads();
    if (wave < e.ntok) {   // Q8_0 of the 32-row block of h for token slot `wave`
        const float v = lane < 32 ? hrow[wave][lane] : 0.0f;
        const float am = half_max(fabsf(v));
        const float d = q8_scale(am);
        const float id = q8_inv(d);
        const int c = e.base + wave;
        if (lane < 32) hq[size_t(c) * ff + rb * 32 + lane] = int8_t(q8_code(v, id));
        if (lane == 0) hd[size_t(c) * (ff / kQ8) + rb] = f16_round(d);
    }
}

// Down with per-slot outputs: workgroup (x, u) takes output rows 4x .. 4x + 3 (one per wave) of entry
// u; yh[tok][slot] as k_hits_down writes it.
__global__ void __launch_bounds__(256) k_gen_down(const DecEntry* __restrict__ ent, const int32_t* __restrict__ n_ent,
                                                  const int8_t* __restrict__ hq, const float* __restrict__ hd, int n,
                                                  int ff, int K, float* __restrict__ yh) {
    if (int(blockIdx.y) >= *n_ent) return;
    const DecEntry e = ent[blockIdx.y];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= n) return;
    const int nbf = ff / kBlock;
    const uint8_t* db = e.blob + 2 * mat_bytes(ff, n);
    float acc[kDecMaxT];
#pragma unroll
    for (int j = 0; j < kDecMaxT; ++j) acc[j] = 0.0f;
    for (int c = lane; c < nbf; c += 64) {
        const uint4 cd = gld_u4(db + (size_t(r) * nbf + c) * 16);
        const float dw = h2f(gld<uint16_t>(db + size_t(n) * nbf * 16 + (size_t(r) * nbf + c) * 2));
        const uint32_t wd[4] = {cd.x, cd.y, cd.z, cd.w};
#pragma unroll
        for (int j = 0; j < kDecMaxT; ++j) {
            if (j >= e.ntok) break;
            const int slot = e.base + j;
            const int4* hp = reinterpret_cast<const int4*>(hq + size_t(slot) * ff + size_t(c) * kBlock);
            int ha[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int4 v = hp[q];
                ha[4 * q] = v.x;
                ha[4 * q + 1] = v.y;
                ha[4 * q + 2] = v.z;
                ha[4 * q + 3] = v.w;
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
            for (int q = 0; q < 8; ++q) s0 = dot4(ha[q], 0x01010101, s0);
#pragma unroll
            for (int q = 8; q < 16; ++q) s1 = dot4(ha[q], 0x01010101, s1);
            const float f = float(q0 - s0) * hd[size_t(slot) * (ff / kQ8) + 2 * c] +
                            float(q1 - s1) * hd[size_t(slot) * (ff / kQ8) + 2 * c + 1];
            acc[j] = acc[j] + f * dw;
        }
    }
#pragma unroll
    for (int j = 0; j < kDecMaxT; ++j) {
        if (j >= e.ntok) break;
        const float y = wave_sum_tree(acc[j]);
        if (lane == 0) yh[(size_t(e.tok[j]) * K + e.slot[j]) * n + r] = y;
    }
}

}  // namespace

// ---------------------------------------------------------------- host side

// scratch: entries, counts, hq, hd for T tokens with K routes (+ the shared expert). The entry array
// has 16 spare slots: the down kernel reads the blob pointers of 4 entries per wave per batch
// before it knows how many entries there are (it uses only those below the count).
static size_t dec_ent_bytes(int T, int K) { return up256(size_t(T * K + 1 + 16) * sizeof(DecEntry)); }
size_t dec_scratch_bytes(int T, int K, int ff) {
    const int S = T * (K + 1);
    return dec_ent_bytes(T, K) + 256 + up256(sizeof(DecComb)) + up256(size_t(S) * ff) +
           up256(size_t(S) * (ff / kQ8) * 4);
}

struct DecScratch {
    DecEntry* ent;
    int32_t* n_ent;
    DecComb* comb;
    int8_t* hq;
    float* hd;
};
static DecScratch dec_carve(void* base, int T, int K, int ff) {
    uint8_t* p = static_cast<uint8_t*>(base);
    DecScratch s;
    s.ent = reinterpret_cast<DecEntry*>(p);
    p += dec_ent_bytes(T, K);
    s.n_ent = reinterpret_cast<int32_t*>(p);
    p += 256;
    s.comb = reinterpret_cast<DecComb*>(p);
    p += up256(sizeof(DecComb));
    s.hq = reinterpret_cast<int8_t*>(p);
    p += up256(size_t(T * (K + 1)) * ff);
    s.hd = reinterpret_cast<float*>(p);
    return s;
}

static int dec_down(const DecScratch& s, int n, int ff, int T, int K, const float* resid, float* out, float* yh,
                    hipStream_t stream, const float* pf = nullptr, int pf_rows = 0, const WinComb& wc = WinComb{}) {
    const int nbf = ff / kBlock;
    const int S = T * (K + 1);                         // compact slots at most (the shared expert's included)
    const int U_max = T * K + 1 < kDecMaxEnt ? T * K + 1 : kDecMaxEnt;   // entries at most
    const size_t smem = size_t(S) * ff + size_t(S) * (ff / kQ8) * 4 + size_t(S) * 8 * 4;
    const size_t hits_smem = std::max(size_t(kHitsDownEnt * kDecMaxT) * (ff + (ff / kQ8) * 4 + 8 * 4),
                                      size_t(kDecMaxHitsT * 8) * 33 * 4 + size_t(kDecMaxHitsT) * 32 * 4);   // (+ the combine's)
#define FRT_DN(NBFV)                                                                                           \
    case NBFV:                                                                                                 \
        if (yh)                                                                                                \
            launch_timed("dec_down", k_hits_down<NBFV>, dim3(n / 8, (U_max + kHitsDownEnt - 1) / kHitsDownEnt),   \
                         dim3(256), hits_smem, stream, s.ent, s.n_ent, s.hq, s.hd, n, ff, K, yh, wc);               \
        else if (T == 1)                                                                                       \
            launch_timed("dec_down", k_dec_down<NBFV, false, true>, dim3(n / 8), dim3(256), smem, stream, s.ent,  \
                         s.n_ent, s.comb, s.hq, s.hd, n, ff, T, K, resid, out, yh, U_max, S, pf, pf_rows);          \
        else                                                                                                   \
            launch_timed("dec_down", k_dec_down<NBFV, false, false>, dim3(n / 8), dim3(256), smem, stream, s.ent, \
                         s.n_ent, s.comb, s.hq, s.hd, n, ff, T, K, resid, out, yh, U_max, S, pf, pf_rows);          \
        break;
    switch (nbf) {
        FRT_DN(4) FRT_DN(8) FRT_DN(10) FRT_DN(16)
        default: return set_error(kErrShape, "decode: ff=%d unsupported (ff/64 in {4,8,10,16})", ff);
    }
#undef FRT_DN
    timing_mark(stream, "dec_down");
    FRT_LAUNCHED("decode down");
    return kOk;
}

// the GEMV shapes instantiated as templates (n / 64 in {16, 32, 40, 48, 64}, ff / 64 in {4, 8, 10, 16})
bool dec_shape_templated(int n, int ff) {
    if (n % 64 || ff % 64) return false;
    const int nb = n / kBlock, nbf = ff / kBlock;
    return (nb == 16 || nb == 32 || nb == 40 || nb == 48 || nb == 64) && (nbf == 4 || nbf == 8 || nbf == 10 || nbf == 16);
}
// the reference's moe_hits envelope (moe_fast.cu:557: n % 512 == 0, ff % 64 == 0, ff <= 4096), n capped here
bool dec_shape_generic(int n, int ff) {
    return n >= 512 && n % 512 == 0 && n <= kGenMaxN && ff >= 64 && ff % 64 == 0 && ff <= kGenMaxFF;
}

int dec_check(int T, int K, int n, int ff) {
    if (T < 1 || T > kDecMaxT) return set_error(kErrShape, "decode: T=%d (1..4)", T);
    if (K < 1 || K > 32 || T * K > 63) return set_error(kErrShape, "decode: K=%d with T=%d (T*K <= 63)", K, T);
    if (n % 64 || ff % 64) return set_error(kErrShape, "decode: n=%d ff=%d (multiples of 64)", n, ff);
    // the instantiated GEMV shapes, checked here so that a refused call launches nothing
    const int nb = n / kBlock, nbf = ff / kBlock;
    if (nb != 16 && nb != 32 && nb != 40 && nb != 48 && nb != 64)
        return set_error(kErrShape, "decode: n=%d unsupported (n/64 in {16,32,40,48,64})", n);
    if (nbf != 4 && nbf != 8 && nbf != 10 && nbf != 16)
        return set_error(kErrShape, "decode: ff=%d unsupported (ff/64 in {4,8,10,16})", ff);
    return kOk;
}

// Whole-window MoE after the router: logits [T][E], gate [T] -> out [T][n] (+ resid).
int dec_moe(const float* logits, const float* gate, int T, int E, int K, const uint8_t* arena, size_t stride,
            const uint8_t* shared_blob, const int8_t* xq, const float* xd, int n, int ff, int32_t* ids, float* wts,
            uint32_t* counts, const float* resid, float* out, void* scratch, hipStream_t stream,
            const float* prefetch) {
    if (int rc = dec_check(T, K, n, ff)) return rc;
    if (E > 1024) return set_error(kErrShape, "decode: E=%d", E);
    const DecScratch s = dec_carve(scratch, T, K, ff);
    const int nb = n / kBlock;
    dim3 g1(ff / 32, T * K + 1);
#define FRT_RG(NBV, VV)                                                                                         \
    if (T == 1)                                                                                                 \
        launch_timed("dec_route_gateup", k_dec_route_gateup<NBV, VV, 1>, g1, dim3(1024), 0, stream, logits, gate, T, \
                     E, K, arena, stride, shared_blob, xq, xd, n, ff, s.hq, s.hd, s.ent, s.n_ent, s.comb, ids, wts,    \
                     counts);                                                                                   \
    else                                                                                                        \
        launch_timed("dec_route_gateup", k_dec_route_gateup<NBV, VV, kDecMaxT>, g1, dim3(1024), 0, stream, logits,  \
                     gate, T, E, K, arena, stride, shared_blob, xq, xd, n, ff, s.hq, s.hd, s.ent, s.n_ent, s.comb, ids, \
                     wts, counts)
#define FRT_RGN(NBV)                       \
    case NBV:                              \
        if (E <= 512) FRT_RG(NBV, 8);      \
        else FRT_RG(NBV, 16);              \
        break;
    switch (nb) {
        FRT_RGN(16) FRT_RGN(32) FRT_RGN(40) FRT_RGN(48) FRT_RGN(64)
        default: return set_error(kErrShape, "decode: n=%d unsupported (n/64 in {16,32,40,48,64})", n);
    }
#undef FRT_RGN
#undef FRT_RG
    timing_mark(stream, "dec_route_gateup");
    return dec_down(s, n, ff, T, K, resid, out, nullptr, stream, prefetch, E);
}

// moe_hits (arch/qwen4exp/moe_fast.hpp:134-142): per-slot expert outputs for the window's hit lists,
// one launch per window of up to kDecMaxHitsT tokens (the reference's kMaxWindow, moe_fast.cu:38),
// each distinct expert's rows read once per four of its tokens.
static int hits_run(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const int8_t* xq, const float* xd,
                    int n, int ff, void* scratch, float* yh, hipStream_t stream, int T, const WinComb& wc) {
    if (T < 1 || T > kDecMaxHitsT || K < 1 || K > 32 || T * K > kHitsMaxItems)
        return set_error(kErrShape, "moe_hits: T=%d K=%d (T <= %d, T*K <= %d per launch)", T, K, kDecMaxHitsT, kHitsMaxItems);
    const bool tmpl = dec_shape_templated(n, ff);
    if (!tmpl && (wc.arrive || !dec_shape_generic(n, ff)))
        return set_error(kErrShape, "moe_hits: n=%d ff=%d (n a multiple of 512 up to %d, ff a multiple of 64 up to %d)",
                         n, ff, kGenMaxN, kGenMaxFF);
    const DecScratch s = dec_carve(scratch, T, K, ff);
    if (hit_ptr) {   // (null: the caller has filled the entry list, dec_window)
        k_hits_group<<<1, kHitsMaxItems, 0, stream>>>(hit_ptr, hit_n, K, T, s.ent, s.n_ent);
        timing_mark(stream, "hits_group");
    }
    if (!tmpl) {   // a shape outside the templated set: the runtime-shape kernels
        const int U_max = T * K < kDecMaxEnt ? T * K : kDecMaxEnt;
        launch_timed("dec_gateup", k_gen_gateup, dim3(ff / 32, U_max), dim3(256), 0, stream, s.ent, s.n_ent, xq, xd, n,
                     ff, s.hq, s.hd);
        FRT_LAUNCHED("moe_hits gate/up");
        launch_timed("dec_down", k_gen_down, dim3((n + 3) / 4, U_max), dim3(256), 0, stream, s.ent, s.n_ent, s.hq, s.hd,
                     n, ff, K, yh);
        FRT_LAUNCHED("moe_hits down");
        return kOk;
    }
    const int nb = n / kBlock;
    dim3 g1(ff / 32, T * K);
#define FRT_GU(NBV) \
    case NBV: k_dec_gateup<NBV><<<g1, 256, 0, stream>>>(s.ent, s.n_ent, xq, xd, n, ff, s.hq, s.hd); break;
    switch (nb) {
        FRT_GU(16) FRT_GU(32) FRT_GU(40) FRT_GU(48) FRT_GU(64)
        default: return set_error(kErrShape, "decode: n=%d unsupported (n/64 in {16,32,40,48,64})", n);
    }
#undef FRT_GU
    timing_mark(stream, "dec_gateup");
    return dec_down(s, n, ff, T, K, nullptr, nullptr, yh, stream, nullptr, 0, wc);
}
int dec_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const int8_t* xq, const float* xd, int n,
             int ff, void* scratch, float* yh, hipStream_t stream, int T) {
    return hits_run(hit_ptr, hit_n, K, xq, xd, n, ff, scratch, yh, stream, T, WinComb{});
}

// A verify window (T <= 8) after routing: ids / wts [T][K], gate [T], the window's Q8_0 input ->
// out [T][n] (+ resid). One moe_hits launch reads each distinct expert once per four of its tokens
// (arch/qwen4exp/moe_fast.cu:195-355), and its down kernel's last workgroup per row group combines.
// Scratch: dec_window_bytes.
size_t dec_window_bytes(int T, int K, int n, int ff) {
    return up256(size_t(T) * (K + 1) * 8) + 256 + up256(size_t(n / 8) * 4) + up256(size_t(T) * (K + 1) * n * 4) +
           dec_scratch_bytes(T, K + 1, ff);
}
int dec_window_fits(int T, int K, int ff) {
    (void)ff;
    // (the window path runs moe_hits over K + 1 slots per token, the shared expert last: K + 1 <= 32)
    return T >= 1 && T <= kDecMaxHitsT && K + 1 <= 32 && T * (K + 1) <= kHitsMaxItems;
}
int dec_window(const float* logits, int E, int32_t* ids, float* wts, uint32_t* counts, const float* gate, int T, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared_blob, const int8_t* xq, const float* xd, int n,
               int ff, const float* resid, float* out, void* scratch, hipStream_t stream) {
    if (!dec_window_fits(T, K, ff) || E < 1 || E > 1024) return set_error(kErrShape, "decode window: T=%d K=%d ff=%d E=%d", T, K, ff, E);
    uint8_t* p = static_cast<uint8_t*>(scratch);
    p += up256(size_t(T) * (K + 1) * 8) + 256;
    int32_t* arrive = reinterpret_cast<int32_t*>(p);
    p += up256(size_t(n / 8) * 4);
    float* yh = reinterpret_cast<float*>(p);
    p += up256(size_t(T) * (K + 1) * n * 4);
    const DecScratch s = dec_carve(p, T, K + 1, ff);
    if (E <= 512)
        launch_timed("win_route", k_win_route<8>, dim3(1), dim3(512), 0, stream, logits, T, E, K, ids, wts, counts,
                     arena, stride, shared_blob, s.ent, s.n_ent, arrive, n / 8);
    else
        launch_timed("win_route", k_win_route<16>, dim3(1), dim3(512), 0, stream, logits, T, E, K, ids, wts, counts,
                     arena, stride, shared_blob, s.ent, s.n_ent, arrive, n / 8);
    FRT_LAUNCHED("decode window routing");
    const WinComb wc{arrive, ids, wts, gate, resid, out, T, K};
    return hits_run(nullptr, nullptr, K + 1, xq, xd, n, ff, p, yh, stream, T, wc);
}

}  // namespace frt
