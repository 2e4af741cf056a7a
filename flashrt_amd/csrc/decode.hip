// Decode / verify-window MoE (T <= 4 tokens): memory-bound fused dequant-GEMVs.
//
// Work list: one entry per distinct expert of the window (each expert's weights are read once for
// every token that selected it, arch/qwen4exp/moe_fast.cu:195-355), in ascending expert id, the
// shared expert last. Entry c-slots (entry u, token j) are numbered compactly (base[u] + j).
//
//   k_dec_route_gateup  per (32 ff rows, entry): every workgroup routes the window itself (top-k
//                 of each token, topk.hpp) and builds the entry list in LDS, so routing costs no
//                 launch; then gate and up rows of every token of its entry, SwiGLU, and Q8_0 of
//                 that 32-row block of h (quant/q2_0/moe_cpu.cpp:43-61 phase A). Workgroup (0, 0)
//                 publishes ids, weights and the entry list.
//   k_dec_gateup  the same body for moe_hits, entries from k_hits_group
//   k_dec_down    per 8 output rows: down rows of every entry, then the weighted sum per token in
//                 expert order plus shared * sigmoid(gate) (moe_cpu.cpp:63-80 phase B and
//                 moe_ref.cu:90-97); or, for moe_hits, the per-slot outputs yh.
//
// Inner product per (row, 64-block, token): the 16 code bytes are read as 4 dwords; (code >> 2s)
// & 0x03030303 lines up with activation dword 4s + w (the planar layout), so 16 v_dot4_i32_i8
// give sum(q * a) for both 32-halves exactly; the -1 offset uses the halves' code sums.
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

constexpr int kDecMaxT = 4;

namespace {

__device__ __forceinline__ float sigmoidf_(float g) { return 1.0f / (1.0f + expf(-g)); }

// ---- the window's routing and its entry list, built in LDS by one 256-thread workgroup: wave t
// routes token t (topk_wave); then wave 0, one lane per selection, orders the distinct experts
// ascending (first occurrences ranked by id), the shared expert last, and numbers the compact slots.
// Needs T * K <= 63. Returns the number of entries (every thread).
struct WinLds {
    DecEntry ent[64];
    int32_t ids[kDecMaxT][32];
    float w[kDecMaxT][32];
    float cand_v[kDecMaxT][64];
    int32_t cand_id[kDecMaxT][64];
    int32_t n_ent;
};

template <int V>
__device__ __forceinline__ int window_entries(const float* __restrict__ logits, const float* __restrict__ gate, int T,
                                              int E, int K, const uint8_t* __restrict__ arena, size_t stride,
                                              const uint8_t* __restrict__ shared_blob, WinLds& L) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (T == 1) {   // one token: the entries are its K experts by ascending id, then the shared expert
        if (wave == 0) {
            const float g = gate[0];
            int sel_id;
            float sel_l, mx, se;
            topk_select<V>(logits, E, K, L.cand_v[0], L.cand_id[0], sel_id, sel_l, mx, se);
            const float w = topk_weight(sel_l, mx, wave_sum_tree(se), K);
            int rank = 0;
            for (int j = 0; j < K; ++j) rank += __builtin_amdgcn_readlane(sel_id, j) < sel_id ? 1 : 0;
            if (lane < K) {
                L.ids[0][lane] = sel_id;
                L.w[0][lane] = w;
                DecEntry& d = L.ent[rank];
                d.blob = arena + size_t(sel_id) * stride;
                d.ntok = 1;
                d.base = rank;
                d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
                d.slot[0] = lane;
                d.slot[1] = d.slot[2] = d.slot[3] = -1;
                d.w[0] = w;
                d.w[1] = d.w[2] = d.w[3] = 0.0f;
            } else if (lane == K) {
                DecEntry& d = L.ent[K];
                d.blob = shared_blob;
                d.ntok = 1;
                d.base = K;
                d.tok[0] = d.tok[1] = d.tok[2] = d.tok[3] = 0;
                d.slot[0] = d.slot[1] = d.slot[2] = d.slot[3] = -1;
                d.w[0] = sigmoidf_(g);
                d.w[1] = d.w[2] = d.w[3] = 0.0f;
                L.n_ent = K + 1;
            }
        }
        __syncthreads();
        return K + 1;
    }
    if (wave < T) topk_wave<V>(logits + size_t(wave) * E, E, K, L.ids[wave], L.w[wave], L.cand_v[wave], L.cand_id[wave]);
    __syncthreads();
    if (wave == 0) {
        const int S = T * K;
        const int e = lane < S ? L.ids[lane / K][lane % K] : 0x7fffffff;
        bool first = lane < S;
        for (int j = 0; j < S; ++j) {
            const int ej = __builtin_amdgcn_readlane(e, j);
            if (j < lane && ej == e) first = false;
        }
        const uint64_t fm = __ballot(first);
        int rank = 0;
        for (int j = 0; j < S; ++j) {
            const int ej = __builtin_amdgcn_readlane(e, j);
            if (((fm >> j) & 1ull) && ej < e) ++rank;
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
            for (int q = nt; q < 4; ++q) {
                d.tok[q] = 0;
                d.slot[q] = -1;
                d.w[q] = 0.0f;
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
            d.w[lane] = lane < T ? sigmoidf_(gate[lane]) : 0.0f;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        const int nt = lane <= U ? L.ent[lane].ntok : 0;
        int tot;
        const int base = wave_excl_scan(nt, &tot);
        if (lane <= U) L.ent[lane].base = base;
        if (lane == 0) L.n_ent = U + 1;
    }
    __syncthreads();
    return L.n_ent;
}

// ---- moe_hits grouping (moe_fast.cu:195-232): distinct blob pointers across the window's hit
// lists, in order of first appearance; no shared expert.
__global__ void k_hits_group(const uint8_t* const* __restrict__ hit_ptr, const int32_t* __restrict__ hit_n, int K, int T,
                             DecEntry* __restrict__ ent, int32_t* __restrict__ n_ent) {
    if (threadIdx.x != 0) return;
    int U = 0, b = 0;
    for (int t = 0; t < T; ++t) {
        const int h = min(hit_n[t], K);
        for (int k = 0; k < h; ++k) {
            const uint8_t* p = hit_ptr[t * K + k];
            int u = 0;
            while (u < U && ent[u].blob != p) ++u;
            if (u == U) {
                DecEntry d{};
                d.blob = p;
                d.ntok = 0;
                for (int j = 0; j < 4; ++j) {
                    d.tok[j] = 0;
                    d.slot[j] = -1;
                    d.w[j] = 0.0f;
                }
                ent[U++] = d;
            }
            DecEntry& d = ent[u];
            d.tok[d.ntok] = t;
            d.slot[d.ntok] = k;
            d.w[d.ntok] = 1.0f;
            ++d.ntok;
        }
    }
    for (int u = 0; u < U; ++u) {
        ent[u].base = b;
        b += ent[u].ntok;
    }
    *n_ent = U;
}

// ---- gate + up for 32 ff rows of one entry. NB = n / 64 blocks per row. 256 threads.
// RPW rows per wave pass (64 / NB when NB divides 64, else 1 with NB <= 64 lanes live).
template <int NB>
__device__ __forceinline__ void gateup_body(const DecEntry& e, const int8_t* __restrict__ xq, const float* __restrict__ xd, int n,
                            int ff, int8_t* __restrict__ hq, float* __restrict__ hd, float (*hrow)[32]) {
    constexpr int RPW = (64 % NB == 0) ? 64 / NB : 1;
    constexpr int PASSES = 8 / RPW;   // 8 rows per wave, 4 waves = 32 rows
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rsub = lane / NB, b = lane % NB;
    const bool live = rsub < RPW;
    const int nb = NB;
    const size_t mb = mat_bytes(ff, n);
    const uint8_t* gcodes = e.blob;
    const uint16_t* gscal = reinterpret_cast<const uint16_t*>(e.blob + size_t(ff) * nb * 16);
    const uint8_t* ucodes = e.blob + mb;
    const uint16_t* uscal = reinterpret_cast<const uint16_t*>(e.blob + mb + size_t(ff) * nb * 16);
    // issue every pass's loads first
    uint4 cg[PASSES], cu[PASSES];
    uint16_t sg[PASSES], su[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int r = blockIdx.x * 32 + wave * 8 + p * RPW + rsub;
        if (live) {
            cg[p] = *reinterpret_cast<const uint4*>(gcodes + (size_t(r) * nb + b) * 16);
            cu[p] = *reinterpret_cast<const uint4*>(ucodes + (size_t(r) * nb + b) * 16);
            sg[p] = gscal[size_t(r) * nb + b];
            su[p] = uscal[size_t(r) * nb + b];
        } else {
            cg[p] = cu[p] = make_uint4(0, 0, 0, 0);
            sg[p] = su[p] = 0;
        }
    }
    // this lane's activation block for each token: 16 dwords, scales, and the halves' code sums
    int xa[kDecMaxT][16];
    float xd0[kDecMaxT], xd1[kDecMaxT];
    int xs0[kDecMaxT], xs1[kDecMaxT];
#pragma unroll
    for (int j = 0; j < kDecMaxT; ++j) {
        if (j < e.ntok && live) {
            const int4* src = reinterpret_cast<const int4*>(xq + size_t(e.tok[j]) * n + b * kBlock);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int4 v = src[q];
                xa[j][4 * q + 0] = v.x;
                xa[j][4 * q + 1] = v.y;
                xa[j][4 * q + 2] = v.z;
                xa[j][4 * q + 3] = v.w;
            }
            xd0[j] = xd[size_t(e.tok[j]) * (n / kQ8) + 2 * b];
            xd1[j] = xd[size_t(e.tok[j]) * (n / kQ8) + 2 * b + 1];
            int s0 = 0, s1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) s0 = dot4(xa[j][i], 0x01010101, s0);
#pragma unroll
            for (int i = 8; i < 16; ++i) s1 = dot4(xa[j][i], 0x01010101, s1);
            xs0[j] = s0;
            xs1[j] = s1;
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) xa[j][i] = 0;
            xd0[j] = xd1[j] = 0.0f;
            xs0[j] = xs1[j] = 0;
        }
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const uint32_t wg[4] = {cg[p].x, cg[p].y, cg[p].z, cg[p].w};
        const uint32_t wu[4] = {cu[p].x, cu[p].y, cu[p].z, cu[p].w};
        const float dg = h2f(sg[p]), du = h2f(su[p]);
        float ag[kDecMaxT], au[kDecMaxT];
#pragma unroll
        for (int j = 0; j < kDecMaxT; ++j) ag[j] = au[j] = 0.0f;
        // integer dots per token and half
#pragma unroll
        for (int j = 0; j < kDecMaxT; ++j) {
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
        // sum over the row's NB lanes (DPP pairwise tree); the total lands in the group's last lane
#pragma unroll
        for (int j = 0; j < kDecMaxT; ++j) {
            if (j >= e.ntok) continue;
            float a = ag[j], c = au[j];
            bool writer;
            if (RPW > 1) {
                a = group_sum<NB>(a);
                c = group_sum<NB>(c);
                writer = live && b == NB - 1;
            } else {
                a = wave_sum_tree(a);
                c = wave_sum_tree(c);
                writer = lane == 0;
            }
            if (writer) hrow[j][wave * 8 + p * RPW + rsub] = a / (1.0f + expf(-a)) * c;
        }
    }
    __syncthreads();
    // Q8_0 of the 32-row block of h for each token: wave w < ntok, lanes 0..31
    if (wave < e.ntok) {   // the whole wave takes part in the DPP max; lanes 0..31 hold the block
        const float v = lane < 32 ? hrow[wave][lane] : 0.0f;
        const float am = half_max(fabsf(v));
        const float d = q8_scale(am);
        const float id = q8_inv(d);
        const int c = e.base + wave;
        if (lane < 32) hq[size_t(c) * ff + blockIdx.x * 32 + lane] = int8_t(q8_code(v, id));
        if (lane == 0) hd[size_t(c) * (ff / kQ8) + blockIdx.x] = f16_round(d);
    }
}

template <int NB>
__global__ void __launch_bounds__(256) k_dec_gateup(const DecEntry* __restrict__ ent, const int32_t* __restrict__ n_ent,
                                                    const int8_t* __restrict__ xq, const float* __restrict__ xd, int n,
                                                    int ff, int8_t* __restrict__ hq, float* __restrict__ hd) {
    __shared__ float hrow[kDecMaxT][32];
    if (int(blockIdx.y) >= *n_ent) return;
    const DecEntry e = ent[blockIdx.y];
    gateup_body<NB>(e, xq, xd, n, ff, hq, hd, hrow);
}

template <int NB, int V>
__global__ void __launch_bounds__(256) k_dec_route_gateup(const float* __restrict__ logits,
                                                          const float* __restrict__ gate, int T, int E, int K,
                                                          const uint8_t* __restrict__ arena, size_t stride,
                                                          const uint8_t* __restrict__ shared_blob,
                                                          const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                          int n, int ff, int8_t* __restrict__ hq,
                                                          float* __restrict__ hd, DecEntry* __restrict__ ent_out,
                                                          int32_t* __restrict__ n_ent_out, int32_t* __restrict__ ids,
                                                          float* __restrict__ wts, uint32_t* counts) {
    __shared__ WinLds L;
    __shared__ float hrow[kDecMaxT][32];
    const int U1 = window_entries<V>(logits, gate, T, E, K, arena, stride, shared_blob, L);
    if (blockIdx.x == 0 && blockIdx.y == 0) {
        for (int i = threadIdx.x; i < U1 * int(sizeof(DecEntry) / 4); i += blockDim.x)
            reinterpret_cast<int32_t*>(ent_out)[i] = reinterpret_cast<const int32_t*>(L.ent)[i];
        if (threadIdx.x < T * K) {
            const int t = threadIdx.x / K, k = threadIdx.x % K;
            ids[t * K + k] = L.ids[t][k];
            wts[t * K + k] = L.w[t][k];
            if (counts) atomicAdd(counts + L.ids[t][k], 1u);
        }
        if (threadIdx.x == 0) *n_ent_out = U1;
    }
    if (int(blockIdx.y) >= U1) return;
    const DecEntry e = L.ent[blockIdx.y];
    gateup_body<NB>(e, xq, xd, n, ff, hq, hd, hrow);
}

// ---- down for 8 output rows x every entry, then the combine. NBF = ff / 64 (8 lanes per row
// when ff = 512). 256 threads; wave w takes entries w, w + 4, ...
template <int NBF>
__global__ void __launch_bounds__(256) k_dec_down(const DecEntry* ent, const int32_t* __restrict__ n_ent,
                                                  const int8_t* __restrict__ hq, const float* __restrict__ hd, int n,
                                                  int ff, int T, int K, const float* __restrict__ resid,
                                                  float* __restrict__ out, float* __restrict__ yh, int U_max,
                                                  int S_max) {
    constexpr int RPP = 64 / NBF;   // rows per wave pass
    constexpr int RD = 8;           // rows per workgroup
    constexpr int PASSES = (RD + RPP - 1) / RPP;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ DecEntry s_ent[64];
    // the entry list, its length and the quantized hidden vectors are independent loads: issue them
    // together (hq/hd for the largest possible slot count S_max), then one barrier
    const int U = *n_ent;
    for (int i = threadIdx.x; i < U_max * int(sizeof(DecEntry) / 4); i += blockDim.x)
        reinterpret_cast<int32_t*>(s_ent)[i] = reinterpret_cast<const int32_t*>(ent)[i];
    int8_t* sh_q = reinterpret_cast<int8_t*>(smem);                        // [S_max][ff]
    float* sh_d = reinterpret_cast<float*>(smem + size_t(S_max) * ff);    // [S_max][ff/32]
    float* sh_y = sh_d + size_t(S_max) * (ff / kQ8);                       // [S_max][RD]
    for (int i = threadIdx.x; i < S_max * ff / 16; i += blockDim.x)
        reinterpret_cast<int4*>(sh_q)[i] = reinterpret_cast<const int4*>(hq)[i];
    for (int i = threadIdx.x; i < S_max * (ff / kQ8); i += blockDim.x) sh_d[i] = hd[i];
    __syncthreads();
    if (U == 0) return;
    ent = s_ent;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rsub = lane / NBF, b = lane % NBF;
    const bool live = rsub < RPP;
    const int r0 = blockIdx.x * RD;
    const int nbf = NBF;
    const size_t dbase = 2 * mat_bytes(ff, n);
    for (int u0 = wave; u0 < U; u0 += 16) {
        // up to 4 entries per batch, all loads issued before use
        uint4 cd[4][PASSES];
        uint16_t sd[4][PASSES];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = u0 + 4 * i;
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int rl = p * RPP + rsub;
                if (u < U && live && rl < RD) {
                    const uint8_t* db = ent[u].blob + dbase;
                    const int r = r0 + rl;
                    cd[i][p] = *reinterpret_cast<const uint4*>(db + (size_t(r) * nbf + b) * 16);
                    sd[i][p] = reinterpret_cast<const uint16_t*>(db + size_t(n) * nbf * 16)[size_t(r) * nbf + b];
                } else {
                    cd[i][p] = make_uint4(0, 0, 0, 0);
                    sd[i][p] = 0;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = u0 + 4 * i;
            if (u >= U) break;
            const DecEntry& e = ent[u];
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int rl = p * RPP + rsub;
                const uint32_t wd[4] = {cd[i][p].x, cd[i][p].y, cd[i][p].z, cd[i][p].w};
                const float dw = h2f(sd[i][p]);
                for (int j = 0; j < e.ntok; ++j) {
                    const int c = e.base + j;
                    float part = 0.0f;
                    if (live && rl < RD) {
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
                    if (live && b == 0 && rl < RD) sh_y[c * RD + rl] = part;
                }
            }
        }
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
    // combine: token t, row rl; routed entries in order (ascending expert), then the shared expert
    for (int i = threadIdx.x; i < T * RD; i += blockDim.x) {
        const int t = i / RD, rl = i % RD;
        float acc = 0.0f;
        for (int u = 0; u < U - 1; ++u) {
            const DecEntry& e = ent[u];
            for (int j = 0; j < e.ntok; ++j)
                if (e.tok[j] == t) {
                    const float p = e.w[j] * sh_y[(e.base + j) * RD + rl];
                    acc = acc + p;
                }
        }
        const DecEntry& sh = ent[U - 1];
        const float p = sh_y[(sh.base + t) * RD + rl] * sh.w[t];
        float o = acc + p;
        if (resid) o = resid[size_t(t) * n + r0 + rl] + o;
        out[size_t(t) * n + r0 + rl] = o;
    }
}

}  // namespace

// ---------------------------------------------------------------- host side

// scratch: entries, counts, hq, hd for T tokens with K routes (+ the shared expert)
size_t dec_scratch_bytes(int T, int K, int ff) {
    const int S = T * (K + 1);
    return up256(size_t(T * K + 1) * sizeof(DecEntry)) + 256 + up256(size_t(S) * ff) + up256(size_t(S) * (ff / kQ8) * 4);
}

struct DecScratch {
    DecEntry* ent;
    int32_t* n_ent;
    int8_t* hq;
    float* hd;
};
static DecScratch dec_carve(void* base, int T, int K, int ff) {
    uint8_t* p = static_cast<uint8_t*>(base);
    DecScratch s;
    s.ent = reinterpret_cast<DecEntry*>(p);
    p += up256(size_t(T * K + 1) * sizeof(DecEntry));
    s.n_ent = reinterpret_cast<int32_t*>(p);
    p += 256;
    s.hq = reinterpret_cast<int8_t*>(p);
    p += up256(size_t(T * (K + 1)) * ff);
    s.hd = reinterpret_cast<float*>(p);
    return s;
}

static int dec_down(const DecScratch& s, int n, int ff, int T, int K, const float* resid, float* out, float* yh,
                    hipStream_t stream) {
    const int nbf = ff / kBlock;
    const int S = T * (K + 1);                         // compact slots at most (the shared expert's included)
    const int U_max = T * K + 1 < 64 ? T * K + 1 : 64;   // entries at most
    const size_t smem = size_t(S) * ff + size_t(S) * (ff / kQ8) * 4 + size_t(S) * 8 * 4;
#define FRT_DN(NBFV)                                                                                           \
    case NBFV:                                                                                                 \
        k_dec_down<NBFV><<<n / 8, 256, smem, stream>>>(s.ent, s.n_ent, s.hq, s.hd, n, ff, T, K, resid, out, yh,  \
                                                       U_max, S);                                               \
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

int dec_check(int T, int K, int n, int ff) {
    if (T < 1 || T > kDecMaxT) return set_error(kErrShape, "decode: T=%d (1..4)", T);
    if (K < 1 || K > 32 || T * K > 63) return set_error(kErrShape, "decode: K=%d with T=%d (T*K <= 63)", K, T);
    if (n % 64 || ff % 64 || n % 8 || ff % 32) return set_error(kErrShape, "decode: n=%d ff=%d", n, ff);
    return kOk;
}

// Whole-window MoE after the router: logits [T][E], gate [T] -> out [T][n] (+ resid).
int dec_moe(const float* logits, const float* gate, int T, int E, int K, const uint8_t* arena, size_t stride,
            const uint8_t* shared_blob, const int8_t* xq, const float* xd, int n, int ff, int32_t* ids, float* wts,
            uint32_t* counts, const float* resid, float* out, void* scratch, hipStream_t stream) {
    if (int rc = dec_check(T, K, n, ff)) return rc;
    if (E > 1024) return set_error(kErrShape, "decode: E=%d", E);
    const DecScratch s = dec_carve(scratch, T, K, ff);
    const int nb = n / kBlock;
    dim3 g1(ff / 32, T * K + 1);
#define FRT_RG(NBV, VV)                                                                                         \
    k_dec_route_gateup<NBV, VV><<<g1, 256, 0, stream>>>(logits, gate, T, E, K, arena, stride, shared_blob, xq, xd, \
                                                        n, ff, s.hq, s.hd, s.ent, s.n_ent, ids, wts, counts)
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
    return dec_down(s, n, ff, T, K, resid, out, nullptr, stream);
}

// moe_hits (arch/qwen4exp/moe_fast.hpp:134-142): per-slot expert outputs for the window's hit lists.
int dec_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const int8_t* xq, const float* xd, int n,
             int ff, void* scratch, float* yh, hipStream_t stream, int T) {
    if (int rc = dec_check(T, K, n, ff)) return rc;
    const DecScratch s = dec_carve(scratch, T, K, ff);
    k_hits_group<<<1, 64, 0, stream>>>(hit_ptr, hit_n, K, T, s.ent, s.n_ent);
    timing_mark(stream, "hits_group");
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
    return dec_down(s, n, ff, T, K, nullptr, nullptr, yh, stream);
}

}  // namespace frt
