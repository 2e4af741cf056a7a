// Top-k routing of one token by one wave64, and the canonical RMS scale, shared by the decode
// and prefill kernels.
//
// Selection (arch/qwen4exp/moe_ref.cu:21-77 semantics; tests/test_route_topk.cpp:52-55 defines the
// order): rank by logit descending, ties to the lower expert id (topk_select below).
// Weights (moe_ref.cu:146-164): p = exp(l - max) / sum_e exp(l_e - max), w_k = p_k / max(sum of the
// selected p in rank order, 2^-14). The sum over all experts is taken in float (pairwise tree); the
// reference's double sum enters the weights only through the rounding of p (the common factor
// cancels in w), which stays within the 1e-6 relative bound.
#pragma once

#include "common.hpp"

namespace frt {

template <int V>
__device__ __forceinline__ void cas_desc(float (&v)[V], int (&id)[V], int i, int j) {
    const bool sw = v[j] > v[i] || (v[j] == v[i] && id[j] < id[i]);
    const float tv = sw ? v[j] : v[i], uv = sw ? v[i] : v[j];
    const int ti = sw ? id[j] : id[i], ui = sw ? id[i] : id[j];
    v[i] = tv;
    v[j] = uv;
    id[i] = ti;
    id[j] = ui;
}

// odd-even transposition rounds (V rounds of disjoint compare-exchanges) sort V values
template <int V>
__device__ __forceinline__ void sort_desc(float (&v)[V], int (&id)[V]) {
#pragma unroll
    for (int r = 0; r < V; ++r)
#pragma unroll
        for (int i = r & 1; i + 1 < V; i += 2) cas_desc<V>(v, id, i, i + 1);
}

// Value of lane (lane ^ j) for j in {1, 2, 4, 8, 16, 32}: DPP (quad permutations, the half-row
// mirror, row rotation by 8) and the gfx950 permlane swaps; no LDS traffic.
template <int J>
__device__ __forceinline__ int lane_xor(int v) {
    if constexpr (J == 1) return __builtin_amdgcn_mov_dpp(v, kDppXor1, 0xF, 0xF, true);
    else if constexpr (J == 2) return __builtin_amdgcn_mov_dpp(v, kDppXor2, 0xF, 0xF, true);
    else if constexpr (J == 4) {   // i ^ 4 = the quad reversal of the half-row mirror (7 - i within 8)
        const int m = __builtin_amdgcn_mov_dpp(v, kDppHalfMirror, 0xF, 0xF, true);
        return __builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, true);   // quad_perm [3,2,1,0]
    } else if constexpr (J == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true);   // row_ror:8
    else if constexpr (J == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (threadIdx.x & 16) ? int(r[0]) : int(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & 32) ? int(r[0]) : int(r[1]);
    }
}

// one compare-exchange stage of a bitonic network over the 64 lanes, order: logit descending,
// expert id ascending on equal logits
template <int K2, int J>
__device__ __forceinline__ void bitonic_stage(float& v, int& id) {
    const int lane = threadIdx.x & 63;
    const float pv = __builtin_bit_cast(float, lane_xor<J>(__builtin_bit_cast(int, v)));
    const int pid = lane_xor<J>(id);
    const bool pbetter = pv > v || (pv == v && pid < id);
    const bool lower = (lane & J) == 0, desc = (lane & K2) == 0;
    const bool take = (lower == desc) ? pbetter : !pbetter;
    v = take ? pv : v;
    id = take ? pid : id;
}

// sorts one (logit, id) pair per lane across the wave: lane 0 gets the best
__device__ __forceinline__ void bitonic64(float& v, int& id) {
    bitonic_stage<2, 1>(v, id);
    bitonic_stage<4, 2>(v, id);
    bitonic_stage<4, 1>(v, id);
    bitonic_stage<8, 4>(v, id);
    bitonic_stage<8, 2>(v, id);
    bitonic_stage<8, 1>(v, id);
    bitonic_stage<16, 8>(v, id);
    bitonic_stage<16, 4>(v, id);
    bitonic_stage<16, 2>(v, id);
    bitonic_stage<16, 1>(v, id);
    bitonic_stage<32, 16>(v, id);
    bitonic_stage<32, 8>(v, id);
    bitonic_stage<32, 4>(v, id);
    bitonic_stage<32, 2>(v, id);
    bitonic_stage<32, 1>(v, id);
    bitonic_stage<64, 32>(v, id);
    bitonic_stage<64, 16>(v, id);
    bitonic_stage<64, 8>(v, id);
    bitonic_stage<64, 4>(v, id);
    bitonic_stage<64, 2>(v, id);
    bitonic_stage<64, 1>(v, id);
}

// exclusive prefix sum of an int over the 64 lanes (and the total): DPP row shifts within each row
// of 16, then row broadcasts across rows
__device__ __forceinline__ int wave_excl_scan(int c, int* total) {
    int x = c;
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, kDppBcast15, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, kDppBcast31, 0xC, 0xF, false);
    *total = __builtin_amdgcn_readlane(x, 63);
    return x - c;
}

// Order key of a logit: unsigned comparison of keys is float comparison of logits, with -0 and +0
// equal (for finite and infinite values; NaN is not a logit). Key 0 is below every logit and marks
// an empty lane.
__device__ __forceinline__ uint32_t logit_key(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u = u == 0x80000000u ? 0u : u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The largest t < 2^12 with at least K lanes holding key >= t << 20 (K >= 1; 0 when fewer than K
// lanes hold a nonzero key): a lower bound on the K-th largest key, found two bits at a time from
// the top by ballot counts over the keys' upper 12 bits (sign, exponent, 3 mantissa bits); uniform.
__device__ __forceinline__ uint32_t wave_kth_key_hi(uint32_t key, int K) {
    const uint32_t kh = key >> 20;
    uint32_t t = 0;
#pragma unroll
    for (int b = 10; b >= 0; b -= 2) {
        const uint32_t c1 = t | (1u << b), c2 = t | (2u << b), c3 = t | (3u << b);
        const int n1 = __popcll(__ballot(kh >= c1)), n2 = __popcll(__ballot(kh >= c2)),
                  n3 = __popcll(__ballot(kh >= c3));
        t = n3 >= K ? c3 : n2 >= K ? c2 : n1 >= K ? c1 : t;
    }
    return t;
}

// Number of lanes below this one whose bit is set in m.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0));
}

// Top-K (K <= 64) of one token's E <= 64 V logits by one wave. cand: 64 floats + 64 ints of LDS
// scratch for this wave. On return lane k < K holds the k-th selection (sel_id, sel_l) in rank
// order; mx is the largest logit and se this lane's share of sum_e exp(l_e - mx).
// Method: lane l holds experts V l .. V l + V - 1. The K best lane maxima (bitonic sort of the 64
// lane maxima) are K distinct logits, so every member of the top K ranks at or above the K-th of
// them; the (few) logits that do are compacted and sorted. Should more than 64 tie there (coarse,
// heavily tied logits), K rounds of wave maxima over the lanes' sorted lists do the selection.
template <int V>
__device__ __forceinline__ void topk_select(const float* __restrict__ l, int E, int K, float* cand_v, int* cand_id,
                                           int& sel_id, float& sel_l, float& mx, float& se) {
    const int lane = threadIdx.x & 63;
    float v[V];
    if (E == 64 * V) {
        const float4* l4 = reinterpret_cast<const float4*>(l + V * lane);
#pragma unroll
        for (int i = 0; i < V / 4; ++i) {
            const float4 q = l4[i];
            v[4 * i] = q.x;
            v[4 * i + 1] = q.y;
            v[4 * i + 2] = q.z;
            v[4 * i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = V * lane + i < E ? l[V * lane + i] : -INFINITY;
    }
    // lane maximum (first index on ties: the lowest expert id of the lane)
    float lm = v[0];
    int li = V * lane;
#pragma unroll
    for (int i = 1; i < V; ++i)
        if (v[i] > lm) {
            lm = v[i];
            li = V * lane + i;
        }
    float sv = lm;
    int sid = li;
    bitonic64(sv, sid);
    mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), 0));
    const float tv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), K - 1));
    const int tid = __builtin_amdgcn_readlane(sid, K - 1);
    se = 0.0f;
    int c = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int e = V * lane + i;
        if (e < E) se += expf(v[i] - mx);
        c += (v[i] > tv || (v[i] == tv && e <= tid)) ? 1 : 0;
    }
    int C;
    int pos = wave_excl_scan(c, &C);
    if (C <= 64) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int e = V * lane + i;
            if (v[i] > tv || (v[i] == tv && e <= tid)) {
                cand_v[pos] = v[i];
                cand_id[pos] = e;
                ++pos;
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        // rank of candidate `lane` among the C candidates (lane j's values read with readlane),
        // then scatter by rank
        const float cv = lane < C ? cand_v[lane] : -INFINITY;
        const int ci = lane < C ? cand_id[lane] : 0x7fffffff;
        int rank = 0;
        for (int j = 0; j < C; ++j) {
            const float ov = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), j));
            const int oi = __builtin_amdgcn_readlane(ci, j);
            rank += (ov > cv || (ov == cv && oi < ci)) ? 1 : 0;
        }
        __builtin_amdgcn_wave_barrier();
        if (lane < C && rank < K) {
            cand_v[rank] = cv;
            cand_id[rank] = ci;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        sel_l = lane < K ? cand_v[lane] : 0.0f;
        sel_id = lane < K ? cand_id[lane] : 0;
        return;
    }
    // heavily tied logits: K rounds over the lanes' sorted lists
    int id[V];
#pragma unroll
    for (int i = 0; i < V; ++i) id[i] = V * lane + i;
    sort_desc<V>(v, id);
    sel_id = 0;
    sel_l = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float m = wave_max(v[0]);
        const uint64_t b = __ballot(v[0] == m);
        const int win = __ffsll((long long)b) - 1;
        const int sel = __builtin_amdgcn_readlane(id[0], win);
        if (lane == win) {
#pragma unroll
            for (int i = 0; i + 1 < V; ++i) {
                v[i] = v[i + 1];
                id[i] = id[i + 1];
            }
            v[V - 1] = -INFINITY;
        }
        if (lane == k) {
            sel_id = sel;
            sel_l = m;
        }
    }
}

// The K weights from a selection (lane k holds the k-th), moe_ref.cu:146-164: p = exp(l - mx) / S
// with S the sum over all experts; w = p / max(sum of the p in rank order, 2^-14).
__device__ __forceinline__ float topk_weight(float sel_l, float mx, float S, int K) {
    const int lane = threadIdx.x & 63;
    float p = 0.0f;
    if (lane < K) p = expf(sel_l - mx) / S;
    float ws = 0.0f;
    for (int k = 0; k < K; ++k) ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), k));
    ws = fmaxf(ws, 6.103515625e-5f);
    return p / ws;
}

// The K weights when E <= 16384 (lane k holds the k-th selection): the selected p are at least
// p_1 = 1 / sum_e exp(l_e - mx) >= 1 / E > 2^-14, so the clamp of moe_ref.cu:146-164 never applies
// and the common factor 1 / sum cancels: w_k = e_k / sum_j e_j with e = exp(l - mx), the sum over
// the selection in rank order. (Against p / sum p with p rounded to float first, this differs by a
// few float roundings, far inside the 1e-6 relative bound.)
__device__ __forceinline__ float topk_weight_sel(float sel_l, float mx, int K) {
    const int lane = threadIdx.x & 63;
    const float e = lane < K ? expf(sel_l - mx) : 0.0f;
    float ws = 0.0f;
    for (int k = 0; k < K; ++k) ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), k));
    return e / ws;
}

// One token by one wave: ids/wts [K] written by lanes 0..K-1; returns lane k's id.
template <int V>
__device__ __forceinline__ int topk_wave(const float* __restrict__ l, int E, int K, int32_t* ids, float* wts,
                                         float* cand_v, int* cand_id) {
    int sel_id;
    float sel_l, mx, se;
    topk_select<V>(l, E, K, cand_v, cand_id, sel_id, sel_l, mx, se);
    const float S = wave_sum_tree(se);
    const float w = topk_weight(sel_l, mx, S, K);
    if ((threadIdx.x & 63) < K) {
        ids[threadIdx.x & 63] = sel_id;
        wts[threadIdx.x & 63] = w;
    }
    return sel_id;
}

// The same selection as topk_wave by ballots in place of the bitonic sort (route1_wave's method):
// a lower bound on the K-th largest lane maximum (ballot counts over the keys' upper 12 bits) makes
// every member of the top K a candidate; the candidates, compacted in ascending id, are ranked by
// logit (ties: lower id first) and scattered by rank. The weights are topk_weight_sel's (the max is
// the rank-0 logit). More than 64 candidates (heavily tied logits) falls back to topk_wave.
// cand_v / cand_id: 128 entries each (64 candidates and one junk slot per lane).
template <int V>
__device__ __forceinline__ int topk_wave_fast(const float* __restrict__ l, int E, int K, int32_t* ids, float* wts,
                                              float* cand_v, int* cand_id) {
    const int lane = threadIdx.x & 63;
    float v[V];
    if (E == 64 * V) {
        const float4* l4 = reinterpret_cast<const float4*>(l + V * lane);
#pragma unroll
        for (int i = 0; i < V / 4; ++i) {
            const float4 q = l4[i];
            v[4 * i] = q.x;
            v[4 * i + 1] = q.y;
            v[4 * i + 2] = q.z;
            v[4 * i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = l[min(V * lane + i, E - 1)];   // past E: masked by the keys
    }
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
    if (C > 64) return topk_wave<V>(l, E, K, ids, wts, cand_v, cand_id);
#pragma unroll
    for (int i = 0; i < V; ++i) {   // branch-free compaction: a non-candidate goes to junk slot 64 + lane
        const bool is_c = key[i] != 0u && key[i] >= t1;
        const int slot = is_c ? pos : 64 + lane;
        cand_v[slot] = v[i];
        cand_id[slot] = V * lane + i;
        pos += int(is_c);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const bool cl = lane < C;
    const float cv = cl ? cand_v[lane] : 0.0f;
    const int ci = cl ? cand_id[lane] : 0x7fffffff;
    int rank = 0;   // candidates ahead: higher logit, or equal and lower id (= lower slot)
    for (int j = 0; j < C; ++j) {
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), j));
        rank += int(o > cv || (o == cv && j < lane));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (cl && rank < K) {
        cand_v[rank] = cv;
        cand_id[rank] = ci;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const float sel_l = lane < K ? cand_v[lane] : 0.0f;
    const int sel_id = lane < K ? cand_id[lane] : 0;
    const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sel_l), 0));
    const float w = topk_weight_sel(sel_l, mx, K);
    if (lane < K) {
        ids[lane] = sel_id;
        wts[lane] = w;
    }
    return sel_id;
}

// ---- Top-K of one token by a group of 4 waves (q = 0..3 the wave's index in the group), for
// latency: the same selection and order as topk_select, with the two ranking passes split over the
// group. Lane l of every wave loads experts V l .. V l + V - 1 (the same data in all 4 waves).
//   1. rank of each lane maximum among the 64 (wave q compares against lanes 16 q .. 16 q + 15;
//      the 4 partial counts meet in LDS); the lane maximum of rank K - 1 is the threshold tv.
//   2. the logits that rank at or above tv are the candidates (at least K, typically a few more);
//      wave 0 compacts them into LDS; each candidate's rank among them is again split over the
//      group; ranks < K are the selection, written in rank order to sel_v / sel_id.
//   (More than 64 candidates, only with coarse heavily tied logits: wave 0 selects by K rounds of
//   wave maxima, as topk_select does.)
// Every wave of the workgroup must call this the same number of times (it holds __syncthreads);
// a group with no token passes active = false. mx (the largest logit) comes back in every wave of
// the group.
struct TopkLds {
    int32_t part[4][64];
    alignas(16) float cand_v[128];     // 64 candidates + one junk slot per lane
    alignas(16) int32_t cand_id[128];
    alignas(16) float sel_v[32];
    alignas(16) int32_t sel_id[32];
    alignas(16) float e[32];   // scratch of the weight step
};

template <int V>
__device__ __forceinline__ void topk_group4(const float* __restrict__ l, int E, int K, int q, bool active,
                                            TopkLds& S, float& mx) {
    const int lane = threadIdx.x & 63;
    if (!active) {   // a group without a token only keeps the workgroup's barrier count (its SIMDs
                     // are shared with the working groups)
        mx = 0.0f;
        __syncthreads();
        __syncthreads();
        __syncthreads();
        __syncthreads();
        return;
    }
    float v[V];
    if (active && E == 64 * V) {
        const float4* l4 = reinterpret_cast<const float4*>(l + V * lane);
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
        for (int i = 0; i < V; ++i) v[i] = (active && V * lane + i < E) ? l[V * lane + i] : -INFINITY;
    }
    float lm = v[0];
    int li = V * lane;
#pragma unroll
    for (int i = 1; i < V; ++i)
        if (v[i] > lm) {
            lm = v[i];
            li = V * lane + i;
        }
    // 1. partial rank of the lane maximum (equal maxima: the lower lane holds the lower id)
    int cnt = 0;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
        const int j = 16 * q + jj;
        const float mj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lm), j));
        cnt += int((mj > lm) | ((mj == lm) & (j < lane)));
    }
    if (active) S.part[q][lane] = cnt;
    __syncthreads();
    const int rank = S.part[0][lane] + S.part[1][lane] + S.part[2][lane] + S.part[3][lane];
    const int kl = __ffsll((long long)__ballot(rank == K - 1)) - 1;
    const int l0 = __ffsll((long long)__ballot(rank == 0)) - 1;
    const float tv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lm), kl));
    const int tid = __builtin_amdgcn_readlane(li, kl);
    mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lm), l0));
    // 2. candidates
    int c = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) c += int((v[i] > tv) | ((v[i] == tv) & (V * lane + i <= tid)));
    int C;
    int pos = wave_excl_scan(c, &C);
    if (active && q == 0 && C <= 64) {   // branch-free compaction: a non-candidate goes to junk slot 64 + lane
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int e = V * lane + i;
            const bool is_c = (v[i] > tv) | ((v[i] == tv) & (e <= tid));
            const int slot = is_c ? pos : 64 + lane;
            S.cand_v[slot] = v[i];
            S.cand_id[slot] = e;
            pos += int(is_c);
        }
    }
    __syncthreads();
    if (C <= 64) {
        const float cv = lane < C ? S.cand_v[lane] : -INFINITY;
        const int ci = lane < C ? S.cand_id[lane] : 0x7fffffff;
        // this wave's 16 candidates as four 16-byte LDS reads of each array (same address in every
        // lane), all issued before the compares; slots >= C are masked
        float ov[16];
        int oi[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 a = reinterpret_cast<const float4*>(S.cand_v + 16 * q)[k];
            const int4 c4 = reinterpret_cast<const int4*>(S.cand_id + 16 * q)[k];
            ov[4 * k] = a.x;
            ov[4 * k + 1] = a.y;
            ov[4 * k + 2] = a.z;
            ov[4 * k + 3] = a.w;
            oi[4 * k] = c4.x;
            oi[4 * k + 1] = c4.y;
            oi[4 * k + 2] = c4.z;
            oi[4 * k + 3] = c4.w;
        }
        int cnt2 = 0;
#pragma unroll
        for (int jj = 0; jj < 16; ++jj)
            cnt2 += int((16 * q + jj < C) & ((ov[jj] > cv) | ((ov[jj] == cv) & (oi[jj] < ci))));
        if (active) S.part[q][lane] = cnt2;
        __syncthreads();
        const int r2 = S.part[0][lane] + S.part[1][lane] + S.part[2][lane] + S.part[3][lane];
        if (active && q == 0 && lane < C && r2 < K) {
            S.sel_v[r2] = cv;
            S.sel_id[r2] = ci;
        }
    } else {
        __syncthreads();
        if (active && q == 0) {   // heavily tied logits: K rounds over the lanes' sorted lists
            int id[V];
#pragma unroll
            for (int i = 0; i < V; ++i) id[i] = V * lane + i;
            sort_desc<V>(v, id);
            for (int k = 0; k < K; ++k) {
                const float m = wave_max(v[0]);
                const uint64_t b = __ballot(v[0] == m);
                const int win = __ffsll((long long)b) - 1;
                const int sel = __builtin_amdgcn_readlane(id[0], win);
                if (lane == win) {
#pragma unroll
                    for (int i = 0; i + 1 < V; ++i) {
                        v[i] = v[i + 1];
                        id[i] = id[i + 1];
                    }
                    v[V - 1] = -INFINITY;
                }
                if (lane == 0) {
                    S.sel_v[k] = m;
                    S.sel_id[k] = sel;
                }
            }
        }
    }
    __syncthreads();
}

// Canonical RMS scale of one token by one wave: chains j = 64 lanes over contiguous L = n / 64
// values, each chain as four contiguous quarters (fmaf(x, x, acc) ascending from 0 in each, so the
// four run side by side) added as (q0 + q1) + (q2 + q3), the adjacent pairwise tree over the chains,
// then r = 1 / sqrt(sum / n + 1e-6) with correctly rounded division and square root.
// xc points at this lane's chain (stride between chain elements: 1).
template <int L>
__device__ __forceinline__ float rms_scale_wave(const float* xc, int n) {
    static_assert(L % 4 == 0, "chains of whole quarters");
    float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < L / 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = fmaf(xc[k * (L / 4) + i], xc[k * (L / 4) + i], q[k]);
    float acc = (q[0] + q[1]) + (q[2] + q[3]);
    acc = wave_sum_tree(acc);
    const float ms = acc / float(n);
    return 1.0f / sqrtf(ms + 1e-6f);
}

}  // namespace frt
