// Pieces of the decode kernels shared by decode.hip (the window kernels) and decode1.hip (the
// single-token persistent layer): the entry list, single-token routing by one wave, and the down
// GEMV rows split into loads and dot products.
#pragma once

#include "common.hpp"
#include "topk.hpp"

namespace frt {

struct DecEntry {
    const uint8_t* blob;   // expert blob (gate | up | down)
    int32_t ntok;          // tokens of the window on this entry, 1..4
    int32_t base;          // first compact slot
    int32_t tok[4];        // token index, ascending
    int32_t slot[4];       // k index of the selection (moe_hits output slot), or -1 for the shared expert
    float w[4];            // routing weight (sigmoid(gate) for the shared expert)
};
static_assert(sizeof(DecEntry) == 64, "DecEntry layout");

constexpr int kDecMaxT = 4;        // tokens per entry, and per routed decode window
constexpr int kDecMaxHitsT = 8;    // tokens per moe_hits launch (the reference's kMaxWindow)
constexpr int kDecMaxEnt = 128;    // entries per launch

namespace {

__device__ __forceinline__ float sigmoidf_(float g) { return 1.0f / (1.0f + expf(-g)); }

// ---- gate/up row sums in the CPU path's float order. matvec_ref (quant/q2_0/q2_0.cpp:119-140) adds a
// row's per-block terms p_b = d_w * (d_a0 s0 + d_a1 s1) one after another from 0, blocks ascending;
// h is then quantized, so a sum off by an ulp can move h across a Q8 code boundary (a pairwise tree
// did on about 3-5% of tokens, up to 2.5e-3 relative in the layer output). Here lane r NB + b
// (r < RPW) holds block b of row r, for M row sets (tokens, or passes over the rows): the gate term
// g[m] and the up term u[m]. Every lane stores its terms in the wave's LDS area buf (M * 128 floats,
// 16-byte aligned); lane c = 2 RPW m + r adds row r's gate terms of set m, lane c + RPW its up terms,
// one after another. Returns (gate sum, up sum) in lane 2 RPW m + r, for m < M and r < RPW (other
// lanes: unspecified). Call with the whole wave active; 2 RPW M <= 64.
// gate/up rows of a 32-row unit over NW waves: 32 / NW rows per wave, RPW = 64 / NB rows per pass (one
// when NB does not divide 64), gu_passes passes
template <int NB> constexpr int gu_rpw() { return (64 % NB == 0) ? 64 / NB : 1; }
template <int NB, int NW> constexpr int gu_passes() { return (32 / NW + gu_rpw<NB>() - 1) / gu_rpw<NB>(); }

template <int NB, int RPW, int M>
__device__ __forceinline__ float2 seq_row_sums(const float (&g)[M], const float (&u)[M], float* buf, int lane) {
    static_assert(2 * RPW * M <= 64 && NB % 4 == 0 && RPW * NB <= 64, "seq_row_sums shape");
#pragma unroll
    for (int m = 0; m < M; ++m) {
        buf[(2 * m) * 64 + lane] = g[m];
        buf[(2 * m + 1) * 64 + lane] = u[m];
    }
    // the wave's LDS operations complete in order; the empty asm keeps the compiler from moving the
    // reads of other lanes' terms above the stores
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    const int m = lane / (2 * RPW), rem = lane % (2 * RPW), gu = rem / RPW, r = rem % RPW;
    float s = 0.0f;
    if (m < M) {
        const float4* q = reinterpret_cast<const float4*>(buf + (2 * m + gu) * 64 + r * NB);
#pragma unroll
        for (int i = 0; i < NB / 4; ++i) {
            const float4 v = q[i];
            s = s + v.x;
            s = s + v.y;
            s = s + v.z;
            s = s + v.w;
        }
    }
    asm volatile("" ::: "memory");   // the next call's stores stay after these reads
    __builtin_amdgcn_wave_barrier();
    const float su = __shfl(s, min(lane + RPW, 63));
    return make_float2(s, su);
}

// ---- the window's routing and its entry list, built in LDS by one 1024-thread workgroup: the 4
// waves of group g route token g together (topk_group4); then wave 0, one lane per selection,
// orders the distinct experts ascending (first occurrences ranked by id), the shared expert last,
// and numbers the compact slots. Needs T * K <= 63. Returns the number of entries (every thread).
// Each token's combine list: its K routed compact slots and weights in ascending expert id, then
// the shared expert's slot and sigmoid(gate) at index K (moe_cpu.cpp:63-80 phase B order).
struct DecComb {
    int32_t slot[kDecMaxT][33];
    float w[kDecMaxT][33];
};

struct WinLds {
    DecEntry ent[64];
    int32_t many;   // the one-wave selection of a single token found more than 64 candidates
    int32_t ids[kDecMaxT][32];
    float w[kDecMaxT][32];
    DecComb comb;
    TopkLds tk[kDecMaxT];
    int32_t n_ent;
};

// The routing and entry list of a single token by one wave, the same selection, weights and
// entries as topk_group4 followed by the single-token entry code below, with ballots in place of
// sorts and barriers:
//   1. lane l holds experts V l .. V l + V - 1; a lower bound on the K-th largest lane maximum (a
//      search over the keys' upper 12 bits by ballot counts) bounds the K-th largest logit from
//      below, so every member of the top K is a candidate; candidates are compacted into LDS in
//      ascending id;
//   2. one candidate per lane: its rank by logit counts the candidates ahead of it (higher key, or
//      equal and lower id); the selection is rank < K, and the entry index is the selection's lane
//      order (ascending id);
//   3. only this workgroup's entry (blockIdx.y) is written, with the rank in slot[0] (w[0]: the
//      selected logit; the weight is formed later, single_weights, while the weight rows load); the
//      ids and logits in rank order go to L.ids and L.w.
// More than 64 candidates (heavily tied logits) sets L.many and writes nothing else; the caller
// then runs the four-wave path. gl is the shared gate logit in lane 0. ALL: every entry is written
// (the persistent single-token layer, where each workgroup needs the whole list).
template <int V, bool ALL = false>
__device__ __forceinline__ void route1_wave(const float (&v)[V], int E, int K, float gl,
                                            const uint8_t* __restrict__ arena, size_t stride,
                                            const uint8_t* __restrict__ shared_blob, WinLds& L) {
    const int lane = threadIdx.x & 63;
    TopkLds& S = L.tk[0];
    uint32_t key[V], mk = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        key[i] = V * lane + i < E ? logit_key(v[i]) : 0u;
        mk = max(mk, key[i]);
    }
    const uint32_t t1 = wave_kth_key_hi(mk, K) << 20;
    int c = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) c += int(key[i] != 0u && key[i] >= t1);
    int C;
    int pos = wave_excl_scan(c, &C);
    if (C > 64) {
        if (lane == 0) L.many = 1;
        return;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {   // branch-free compaction: a non-candidate goes to junk slot 64 + lane
        const bool is_c = key[i] != 0u && key[i] >= t1;
        const int slot = is_c ? pos : 64 + lane;
        S.cand_v[slot] = v[i];
        S.cand_id[slot] = V * lane + i;
        pos += int(is_c);
    }
    const bool cl = lane < C;
    const float cv = cl ? S.cand_v[lane] : 0.0f;
    const int ci = cl ? S.cand_id[lane] : 0x7fffffff;
    // rank among the candidates: those ahead by logit, or equal and lower id (= lower slot); each
    // candidate's logit broadcast from its lane (no LDS round trip per step); float order with
    // -0 == +0 is the keys' order
    int rank = 0;
    for (int j = 0; j < C; ++j) {
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), j));
        rank += int(o > cv || (o == cv && j < lane));
    }
    const bool sel = cl && rank < K;
    const int u = lanes_below(__ballot(sel));   // entry index: ascending expert id
    // Each workgroup needs only its own entry (blockIdx.y); the entries carry the selected logit in
    // w[0] (the gate logit for the shared one) and the rank in slot[0], and the down kernel forms
    // the weights from them. The ids in rank order go to every workgroup's L.ids (published by
    // the workgroups of the first row block).
    const int my = int(blockIdx.y);
    if (sel) {
        L.ids[0][rank] = ci;
        L.w[0][rank] = cv;   // the selected logits in rank order (for the weights)
        if (ALL || u == my) {
            DecEntry& d = L.ent[u];
            d.blob = arena + size_t(ci) * stride;
            d.ntok = 1;
            d.base = u;
            d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
            d.slot[0] = rank;
            d.slot[1] = d.slot[2] = d.slot[3] = -1;
            d.w[0] = cv;
            d.w[1] = d.w[2] = d.w[3] = 0.0f;
        }
    }
    const float g0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gl), 0));
    if (lane == 63) {
        if (ALL || my == K) {
            DecEntry& d = L.ent[K];
            d.blob = shared_blob;
            d.ntok = 1;
            d.base = K;
            d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
            d.slot[0] = d.slot[1] = d.slot[2] = d.slot[3] = -1;
            d.w[0] = g0;
            d.w[1] = d.w[2] = d.w[3] = 0.0f;
        }
        L.n_ent = K + 1;
        L.many = 0;
    }
}

// ---- The same routing of a single token (selection, tie rule, entries and records as
// route1_wave<V, true>) by the 8 waves of a workgroup, for latency: wave w holds experts 64 w + lane
// (E <= 512), one per lane, so each wave's steps are on one value per lane.
//   1. each wave: a lower bound on its own K-th largest key (wave_kth_key_hi); their maximum T is a
//      lower bound on the K-th largest key of all E (a wave with K keys >= t puts K keys >= t in all);
//   2. each wave compacts its keys >= T (every member of the top K) into LDS in ascending id;
//   3. wave 0 takes the candidates, in ascending id, one per lane, and ranks them by logit (ties: the
//      lower id, the lower position) as route1_wave does; more than 64 candidates (heavily tied
//      logits) sets L.many.
// Every wave of the workgroup calls it (it holds barriers). A wave may start as soon as its own
// lanes' logits are in s_lg (each lane reads only the word at its expert); s_lg[E] (the shared gate
// logit) is read by wave 0 after the first barrier.
struct Route8Lds {
    uint32_t t[8];
    int32_t cnt[8];
    float v[8][64];
    int32_t id[8][64];
};
__device__ __forceinline__ void route_8waves(const float* s_lg, int E, int K, const uint8_t* __restrict__ arena,
                                             size_t stride, const uint8_t* __restrict__ shared_blob, WinLds& L,
                                             Route8Lds& Q) {
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6), lane = threadIdx.x & 63;
    const int e = 64 * wave + lane;
    const float v = s_lg[min(e, E - 1)];
    const uint32_t key = e < E ? logit_key(v) : 0u;
    const uint32_t tw = wave_kth_key_hi(key, K) << 20;
    if (lane == 0) Q.t[wave] = tw;
    __syncthreads();
    uint32_t T = Q.t[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) T = max(T, Q.t[w]);
    const bool c = key != 0u && key >= T;
    const uint64_t m = __ballot(c);
    if (c) {
        const int pos = lanes_below(m);
        Q.v[wave][pos] = v;
        Q.id[wave][pos] = e;
    }
    if (lane == 0) Q.cnt[wave] = int(__popcll(m));
    __syncthreads();
    if (wave != 0) return;
    int C = 0, sw = 0, si = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        const int cw = Q.cnt[w];
        if (lane >= C && lane < C + cw) {
            sw = w;
            si = lane - C;
        }
        C += cw;
    }
    if (C > 64) {
        if (lane == 0) L.many = 1;
        return;
    }
    const bool cl = lane < C;
    const float cv = cl ? Q.v[sw][si] : 0.0f;
    const int ci = cl ? Q.id[sw][si] : 0x7fffffff;
    int rank = 0;   // candidates ahead: higher logit, or equal and lower id (= lower position)
    for (int j = 0; j < C; ++j) {
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), j));
        rank += int(o > cv || (o == cv && j < lane));
    }
    const bool sel = cl && rank < K;
    const int u = lanes_below(__ballot(sel));   // entry index: ascending expert id
    if (sel) {
        L.ids[0][rank] = ci;
        L.w[0][rank] = cv;
        DecEntry& d = L.ent[u];
        d.blob = arena + size_t(ci) * stride;
        d.ntok = 1;
        d.base = u;
        d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
        d.slot[0] = rank;
        d.slot[1] = d.slot[2] = d.slot[3] = -1;
        d.w[0] = cv;
        d.w[1] = d.w[2] = d.w[3] = 0.0f;
    }
    if (lane == 63) {
        DecEntry& d = L.ent[K];
        d.blob = shared_blob;
        d.ntok = 1;
        d.base = K;
        d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
        d.slot[0] = d.slot[1] = d.slot[2] = d.slot[3] = -1;
        d.w[0] = s_lg[E];
        d.w[1] = d.w[2] = d.w[3] = 0.0f;
        L.n_ent = K + 1;
        L.many = 0;
    }
}

// after_issue() runs once the routing's own loads are issued (a single token: the logits in wave 0),
// for loads the caller wants in flight during the routing but not waited for before it.
struct NoLoads {
    __device__ void operator()() const {}
};
template <int V, class F = NoLoads>
__device__ __forceinline__ int window_entries(const float* __restrict__ logits, const float* __restrict__ gate, int T,
                                              int E, int K, const uint8_t* __restrict__ arena, size_t stride,
                                              const uint8_t* __restrict__ shared_blob, WinLds& L,
                                              F after_issue = {}) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g = wave >> 2, q = wave & 3;
    const bool active = g < T;
    // shared gate logits, issued with the logits (a plain load: a volatile one is waited for where it
    // is issued); every lane loads (a clamped index, no branch, so no wait is placed at a branch merge)
    const float gl = gate[min(lane, T - 1)];
    float mx;
    if (T == 1) {   // one wave selects; the rest of the workgroup waits at the barrier
        // every wave loads the logits (L1 hits after the first), so no load sits under a branch and
        // no wait is placed at a branch merge ahead of after_issue()'s loads
        float v[V];
        if (E == 64 * V) {
            const float4* l4 = reinterpret_cast<const float4*>(logits + V * lane);
#pragma unroll
            for (int i = 0; i < V / 4; ++i) {
                const float4 f = l4[i];
                v[4 * i] = f.x;
                v[4 * i + 1] = f.y;
                v[4 * i + 2] = f.z;
                v[4 * i + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) v[i] = logits[min(V * lane + i, E - 1)];
        }
        __builtin_amdgcn_sched_barrier(0);
        after_issue();   // issued behind the logits: the wait for them leaves these in flight
        __builtin_amdgcn_sched_barrier(0);
        if (wave == 0) route1_wave<V>(v, E, K, gl, arena, stride, shared_blob, L);
        __syncthreads();
        if (!L.many) {
            return K + 1;
        }
    }
    topk_group4<V>(logits + size_t(active ? g : 0) * E, E, K, q, active, L.tk[active ? g : 0], mx);
    if (T == 1) {   // one token (heavy ties): every entry, in route1_wave's form (logit in w[0], rank in slot[0])
        if (wave == 0) {
            const float sel_l = lane < K ? L.tk[0].sel_v[lane] : 0.0f;
            const int sel_id = lane < K ? L.tk[0].sel_id[lane] : 0x7fffffff;
            int u = 0;
            for (int j = 0; j < K; ++j) u += int(__builtin_amdgcn_readlane(sel_id, j) < sel_id);
            const float g0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gl), 0));
            if (lane < K) {
                L.ids[0][lane] = sel_id;
                L.w[0][lane] = sel_l;
                DecEntry& d = L.ent[u];
                d.blob = arena + size_t(sel_id) * stride;
                d.ntok = 1;
                d.base = u;
                d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
                d.slot[0] = lane;
                d.slot[1] = d.slot[2] = d.slot[3] = -1;
                d.w[0] = sel_l;
                d.w[1] = d.w[2] = d.w[3] = 0.0f;
            } else if (lane == K) {
                DecEntry& d = L.ent[K];
                d.blob = shared_blob;
                d.ntok = 1;
                d.base = K;
                d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
                d.slot[0] = d.slot[1] = d.slot[2] = d.slot[3] = -1;
                d.w[0] = g0;
                d.w[1] = d.w[2] = d.w[3] = 0.0f;
                L.n_ent = K + 1;
            }
        }
        __syncthreads();
        return K + 1;
    }
    if (active && q == 0) {
        const float sel_l = lane < K ? L.tk[g].sel_v[lane] : 0.0f;
        const float w = topk_weight_sel(sel_l, mx, K);
        if (lane < K) {
            L.ids[g][lane] = L.tk[g].sel_id[lane];
            L.w[g][lane] = w;
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int S = T * K;
        const int e = lane < S ? L.ids[lane / K][lane % K] : 0x7fffffff;
        bool first = lane < S;
        int pos = 0;   // earlier selections of the same expert (their tokens come first in the entry)
        for (int j = 0; j < S; ++j) {
            const int ej = __builtin_amdgcn_readlane(e, j);
            if (j < lane && ej == e) {
                first = false;
                ++pos;
            }
        }
        const uint64_t fm = __ballot(first);
        int rank = 0;   // entry of this lane's expert: distinct experts with a smaller id
        int rk = 0;     // position in its token's list: the token's experts with a smaller id
        const int tl = lane / K;
        for (int j = 0; j < S; ++j) {
            const int ej = __builtin_amdgcn_readlane(e, j);
            if (((fm >> j) & 1ull) && ej < e) ++rank;
            if (j / K == tl && ej < e) ++rk;
        }
        const int U = __popcll(fm);
        if (first) {
            DecEntry& d = L.ent[rank];
            d.blob = arena + size_t(e) * stride;
            int nt = 0;
            for (int j = 0; j < S; ++j) {
                const int ej = __builtin_amdgcn_readlane(e, j);
                if (ej == e) {
                    d.tok[nt] = j / K;
                    d.slot[nt] = j % K;
                    d.w[nt] = L.w[j / K][j % K];
                    ++nt;
                }
            }
            d.ntok = nt;
            for (int qq = nt; qq < 4; ++qq) {
                d.tok[qq] = 0;
                d.slot[qq] = -1;
                d.w[qq] = 0.0f;
            }
        }
        if (lane < 4) {   // the shared expert, every token, weight sigmoid(gate)
            DecEntry& d = L.ent[U];
            if (lane == 0) {
                d.blob = shared_blob;
                d.ntok = T;
            }
            d.tok[lane] = lane < T ? lane : 0;
            d.slot[lane] = -1;
            d.w[lane] = lane < T ? sigmoidf_(gl) : 0.0f;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        const int nt = lane <= U ? L.ent[lane].ntok : 0;
        int tot;
        const int base = wave_excl_scan(nt, &tot);
        if (lane <= U) L.ent[lane].base = base;
        if (lane == 0) L.n_ent = U + 1;
        // combine lists: slot = base of the expert's entry + pos; the shared expert's slot is its base + t
        const int eb = __shfl(base, rank, 64);
        const int sb = __builtin_amdgcn_readlane(base, U);
        if (lane < S) {
            L.comb.slot[tl][rk] = eb + pos;
            L.comb.w[tl][rk] = L.w[tl][lane % K];
        }
        if (lane < T) {
            L.comb.slot[lane][K] = sb + lane;
            L.comb.w[lane][K] = sigmoidf_(gl);
        }
    }
    __syncthreads();
    return L.n_ent;
}

// ---- down GEMV rows, split into loads (issued early, into registers) and the dot products, so
// that a batch of down rows is in flight while the kernel stages its other inputs.
// Wave w takes entries u0 + 4 i (i < BATCH) of the list, u0 = w + 4 BATCH b for batch b; each
// of its lanes holds one 64-block of one of the RD = 8 rows r0 .. r0 + 7.
template <int NBF, int BATCH>
struct DownRegs {
    static constexpr int RPP = 64 / NBF;   // rows per wave pass
    static constexpr int RD = 8;           // rows per workgroup
    static constexpr int PASSES = (RD + RPP - 1) / RPP;
    uint4 cd[BATCH][PASSES];
    uint32_t sd[BATCH][PASSES];   // fp16 scale bits, one per register
    uint32_t ok;                  // bit i * PASSES + p: that row load is real (else it counts as 0)
};

// US: entry step between a wave's batch members (the number of waves); LDS_ENT: ent is in LDS
// (read there with clamped indices) rather than in global memory.
template <int NBF, int BATCH, int US = 4, bool LDS_ENT = false>
__device__ __forceinline__ void down_load(const DecEntry* ent, int U, int u0, int r0, int n, int ff,
                                          DownRegs<NBF, BATCH>& R) {
    using D = DownRegs<NBF, BATCH>;
    const int lane = threadIdx.x & 63;
    const int rsub = lane / NBF, b = lane % NBF;
    const bool live = rsub < D::RPP;
    const size_t dbase = 2 * mat_bytes(ff, n);
    // The entries' blob pointers in one vector load (lane i < BATCH: entry u0 + 4 i; lane BATCH:
    // entry 0, which stands in for entries past U; the entry array holds at least 4 BATCH entries,
    // so the load need not wait for U), then every row load, unconditional (clamped entry and row;
    // the ok mask zeroes the invalid ones where they are used), so that they issue back to back.
    // Needs U >= 1.
    const int le = lane < BATCH ? u0 + US * lane : 0;
    const uint64_t bp = LDS_ENT ? reinterpret_cast<uint64_t>(ent[min(le, U - 1)].blob) : gld<uint64_t>(&ent[le].blob);
    const uint64_t b0 = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(bp >> 32)), BATCH))) << 32) |
                        uint32_t(__builtin_amdgcn_readlane(int(uint32_t(bp)), BATCH));
    const uint8_t* db[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        const uint64_t bi = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(bp >> 32)), i))) << 32) |
                            uint32_t(__builtin_amdgcn_readlane(int(uint32_t(bp)), i));
        db[i] = reinterpret_cast<const uint8_t*>(u0 + US * i < U ? bi : b0) + dbase;
    }
    R.ok = 0;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
#pragma unroll
        for (int p = 0; p < D::PASSES; ++p) {
            const int rl = p * D::RPP + rsub;
            if (u0 + US * i < U && live && rl < D::RD) R.ok |= 1u << (i * D::PASSES + p);
            const int r = r0 + min(rl, D::RD - 1);
            const int bb = live ? b : 0;
            R.cd[i][p] = gld_u4_nt(db[i] + (size_t(r) * NBF + bb) * 16);
            R.sd[i][p] = gld<uint16_t>(db[i] + size_t(n) * NBF * 16 + (size_t(r) * NBF + bb) * 2);
        }
    }
}

// down_compute for a single token (entry u's compact slot is u): the same products and sums, with the
// BATCH entries computed side by side (no per-entry reads of the entry list, whose LDS round trips
// would otherwise run one after another)
template <int NBF, int BATCH, int US = 4>
__device__ __forceinline__ void down_compute1(int U, int u0, const DownRegs<NBF, BATCH>& R, const int8_t* sh_q,
                                              const float* sh_d, float* sh_y, int ff) {
    using D = DownRegs<NBF, BATCH>;
    const int lane = threadIdx.x & 63;
    const int rsub = lane / NBF, b = lane % NBF;
    const bool live = rsub < D::RPP;
    float part[BATCH][D::PASSES];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        const int c = min(u0 + US * i, U - 1);
        const int4* hp = reinterpret_cast<const int4*>(sh_q + size_t(c) * ff + (live ? b : 0) * kBlock);
        int ha[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int4 v = hp[q];
            ha[4 * q] = v.x;
            ha[4 * q + 1] = v.y;
            ha[4 * q + 2] = v.z;
            ha[4 * q + 3] = v.w;
        }
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i2 = 0; i2 < 8; ++i2) s0 = dot4(ha[i2], 0x01010101, s0);
#pragma unroll
        for (int i2 = 8; i2 < 16; ++i2) s1 = dot4(ha[i2], 0x01010101, s1);
        const float d0 = sh_d[size_t(c) * (ff / kQ8) + 2 * (live ? b : 0)];
        const float d1 = sh_d[size_t(c) * (ff / kQ8) + 2 * (live ? b : 0) + 1];
#pragma unroll
        for (int p = 0; p < D::PASSES; ++p) {
            const bool ok = (R.ok >> (i * D::PASSES + p)) & 1u;
            const uint32_t wd[4] = {ok ? R.cd[i][p].x : 0u, ok ? R.cd[i][p].y : 0u, ok ? R.cd[i][p].z : 0u,
                                    ok ? R.cd[i][p].w : 0u};
            const float dw = ok ? h2f(uint16_t(R.sd[i][p])) : 0.0f;
            int q0 = 0, q1 = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                q0 = dot4(int(wd[w] & 0x03030303u), ha[w], q0);
                q0 = dot4(int((wd[w] >> 2) & 0x03030303u), ha[4 + w], q0);
                q1 = dot4(int((wd[w] >> 4) & 0x03030303u), ha[8 + w], q1);
                q1 = dot4(int((wd[w] >> 6) & 0x03030303u), ha[12 + w], q1);
            }
            const float f = float(q0 - s0) * d0 + float(q1 - s1) * d1;
            part[i][p] = (live && p * D::RPP + rsub < D::RD) ? f * dw : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < BATCH; ++i)
#pragma unroll
        for (int p = 0; p < D::PASSES; ++p) {
            float v = part[i][p];
            if ((NBF & (NBF - 1)) == 0 && NBF <= 16) {
                v = group_sum<(NBF <= 16 ? NBF : 16)>(v);
            } else {
                float acc = 0.0f;
                for (int q = 0; q < NBF; ++q) acc += __shfl(v, rsub * NBF + q, 64);
                v = acc;
            }
            const int rl = p * D::RPP + rsub;
            if (u0 + US * i < U && live && b == 0 && rl < D::RD) sh_y[(u0 + US * i) * D::RD + rl] = v;
        }
}

// sh_q [S][ff] int8 and sh_d [S][ff/32] are the Q8_0 hidden vectors by compact slot; writes
// sh_y[c * 8 + rl], the down row r0 + rl of slot c (pairwise tree over the row's NBF blocks)
template <int NBF, int BATCH, int US = 4>
__device__ __forceinline__ void down_compute(const DecEntry* ent, int U, int u0, const DownRegs<NBF, BATCH>& R,
                                             const int8_t* sh_q, const float* sh_d, float* sh_y, int ff) {
    using D = DownRegs<NBF, BATCH>;
    const int lane = threadIdx.x & 63;
    const int rsub = lane / NBF, b = lane % NBF;
    const bool live = rsub < D::RPP;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        const int u = u0 + US * i;
        if (u >= U) break;
        const DecEntry& e = ent[u];
#pragma unroll
        for (int p = 0; p < D::PASSES; ++p) {
            const int rl = p * D::RPP + rsub;
            const bool ok = (R.ok >> (i * D::PASSES + p)) & 1u;
            const uint32_t wd[4] = {ok ? R.cd[i][p].x : 0u, ok ? R.cd[i][p].y : 0u, ok ? R.cd[i][p].z : 0u,
                                    ok ? R.cd[i][p].w : 0u};
            const float dw = ok ? h2f(uint16_t(R.sd[i][p])) : 0.0f;
            for (int j = 0; j < e.ntok; ++j) {
                const int c = e.base + j;
                float part = 0.0f;
                if (live && rl < D::RD) {
                    const int4* hp = reinterpret_cast<const int4*>(sh_q + size_t(c) * ff + b * kBlock);
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
                    for (int i2 = 0; i2 < 8; ++i2) s0 = dot4(ha[i2], 0x01010101, s0);
#pragma unroll
                    for (int i2 = 8; i2 < 16; ++i2) s1 = dot4(ha[i2], 0x01010101, s1);
                    const float f = float(q0 - s0) * sh_d[size_t(c) * (ff / kQ8) + 2 * b] +
                                    float(q1 - s1) * sh_d[size_t(c) * (ff / kQ8) + 2 * b + 1];
                    part = f * dw;
                }
                if ((NBF & (NBF - 1)) == 0 && NBF <= 16) {
                    part = group_sum<(NBF <= 16 ? NBF : 16)>(part);
                } else {
                    // segments of NBF lanes: gather the row's partials from its first lane
                    float acc = 0.0f;
                    for (int q = 0; q < NBF; ++q) acc += __shfl(part, rsub * NBF + q, 64);
                    part = acc;
                }
                if (live && b == 0 && rl < D::RD) sh_y[c * D::RD + rl] = part;
            }
        }
    }
}

// A staging copy of count >= 1 elements from global memory to LDS by a workgroup of NT threads,
// split into its loads and its LDS writes, so that a kernel can issue every staging load (and
// other loads) before the first write waits: B elements per thread are staged this way (clamped
// indices, no branches; threads past the end rewrite the last element with its own value), the
// rest (larger windows only) by a plain loop in store(). NT is the workgroup size as a constant:
// blockDim.x is read from the dispatch packet, and a wait for that load would also wait for every
// load issued before it.
template <class T, int B, int NT>
struct Stage {
    T v[B];
    __device__ __forceinline__ void load(const T* __restrict__ src, int count) {
#pragma unroll
        for (int k = 0; k < B; ++k) v[k] = src[min(int(threadIdx.x) + k * NT, count - 1)];
    }
    __device__ __forceinline__ void store(T* dst, const T* __restrict__ src, int count) const {
#pragma unroll
        for (int k = 0; k < B; ++k) dst[min(int(threadIdx.x) + k * NT, count - 1)] = v[k];
        for (int i = int(threadIdx.x) + B * NT; i < count; i += NT) dst[i] = src[i];
    }
};

}  // namespace
}  // namespace frt
