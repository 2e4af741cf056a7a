// Router logits, Q8_0 activation quantization and top-k routing.
//
// Router logits use one canonical float order, shared with the CPU oracle, so that expert ids
// match bit for bit: logit[t][e] = tree over 64 chains, chain j = fmaf over k in [j L, (j+1) L)
// ascending from 0 (L = n / 64), tree s_m(j) = s_{m-1}(j) + s_{m-1}(j + 64 >> m), then + bias[e].
// On the GPU a wave owns one router row: lane j is chain j and the xor butterfly over lanes is
// exactly that tree (float addition is commutative).
//
// Top-k (arch/qwen4exp/moe_ref.cu:21-77 semantics): rank by logit descending, ties to the lower
// expert id; p = exp(l - max) / sum (sum in double); weights p_k / max(sum_k p_k, 2^-14).
#include "common.hpp"

namespace frt {
namespace {

constexpr int kMaxE = 1024;   // experts a routing wave handles (16 logits per lane)

// ---- router GEMV/GEMM: grid (ceil(rows / 8), ceil(T / TT)); 8 waves, one router row each.
// Rows 0..E-1 are the router (bias optional); row E (when gate_w) is the shared expert's gate.
// x tile [TT][n] staged in LDS with each 64-chain padded by one float (conflict-free reads).
template <int L>
__global__ void __launch_bounds__(512) k_router(const float* __restrict__ x, int T, const float* __restrict__ W,
                                                const float* __restrict__ bias, const float* __restrict__ gate_w,
                                                int E, float* __restrict__ logits, float* __restrict__ gate, int TT,
                                                int tok_per_wg) {
    extern __shared__ float xs[];   // [TT][64][L + 1]
    const int n = 64 * L;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 8 + wave;
    const bool is_gate = row == E;
    const bool live = row < E || (is_gate && gate_w);
    const float* w = is_gate ? gate_w : W + size_t(row < E ? row : 0) * n;
    float wr[L];
#pragma unroll
    for (int i = 0; i < L; ++i) wr[i] = live ? w[lane * L + i] : 0.0f;
    const float b = (live && !is_gate && bias) ? bias[row] : 0.0f;
    const int t_begin = blockIdx.y * tok_per_wg, t_end = min(T, t_begin + tok_per_wg);
    for (int t0 = t_begin; t0 < t_end; t0 += TT) {
        const int tn = min(TT, t_end - t0);
        __syncthreads();
        for (int i = threadIdx.x; i < tn * n; i += blockDim.x) {
            const int t = i / n, k = i % n;
            xs[(t * 64 + k / L) * (L + 1) + k % L] = x[size_t(t0 + t) * n + k];
        }
        __syncthreads();
        if (!live) continue;
        for (int t = 0; t < tn; ++t) {
            const float* xc = xs + (t * 64 + lane) * (L + 1);
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < L; ++i) acc = fmaf(wr[i], xc[i], acc);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o, 64);
            if (lane == 0) {
                if (is_gate) gate[t0 + t] = acc;
                else logits[size_t(t0 + t) * E + row] = bias ? acc + b : acc;
            }
        }
    }
}

// ---- Q8_0 of activations: one wave per 2 blocks of 32 (quant/q2_0/q2_0.cpp:93-108).
// xq int8 [rows][n] natural order, xd [rows][n/32]. With xq16: the same codes as fp16 in the
// prefill GEMM's operand order (perm64 below), [rows][n].
__global__ void k_quant_q8(const float* __restrict__ x, int n_blocks, int8_t* __restrict__ xq, float* __restrict__ xd,
                           _Float16* __restrict__ xq16, int n) {
    const int gw = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;   // global wave
    const int lane = threadIdx.x & 63;
    const int blk = gw * 2 + (lane >> 5);
    if (blk >= n_blocks) return;
    const int j = lane & 31;
    const float v = x[size_t(blk) * kQ8 + j];
    float am = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
    const float d = q8_scale(am);
    const float id = q8_inv(d);
    const int q = q8_code(v, id);
    xq[size_t(blk) * kQ8 + j] = int8_t(q);
    if (j == 0) xd[blk] = f16_round(d);
    if (xq16) {
        // position of element e of a 64-block in the permuted order: inverse of perm64_elem
        const int e = (blk & 1) * 32 + j;   // element within the 64-block
        const int s = e >> 4, g = (e >> 2) & 3, c = e & 3;
        const int h = s >> 1, ci = c == 0 ? 0 : c == 1 ? 2 : c == 2 ? 1 : 3;
        const int slot = (s & 1) * 4 + ci;
        const size_t base = size_t(blk >> 1) * kBlock;
        xq16[base + h * 32 + g * 8 + slot] = _Float16(float(q));
    }
}

// ---- top-k for one token by one wave. Keys: orderable logit bits << 32 | (0xffffffff - id), so
// the wave maximum is the largest logit with the lowest id on ties.
__device__ inline uint64_t route_key(float l, int e) {
    uint32_t b = __builtin_bit_cast(uint32_t, l);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (uint64_t(b) << 32) | uint64_t(0xffffffffu - uint32_t(e));
}
__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor(uint32_t(v), o, 64), hi = __shfl_xor(uint32_t(v >> 32), o, 64);
        const uint64_t w = (uint64_t(hi) << 32) | lo;
        v = w > v ? w : v;
    }
    return v;
}
__device__ inline double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Writes ids/wts [K] for the token's logits l [E]; returns (in every lane) nothing; sel_out (LDS,
// optional) gets the ids too.
template <int V>
__device__ void topk_wave(const float* __restrict__ l, int E, int K, int32_t* __restrict__ ids, float* __restrict__ wts,
                          uint32_t* counts, uint32_t* tail, bool in_tail) {
    const int lane = threadIdx.x & 63;
    float v[V];
    uint64_t key[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int e = 64 * i + lane;
        v[i] = e < E ? l[e] : -INFINITY;
        key[i] = e < E ? route_key(v[i], e) : 0;
    }
    // selection: K rounds of the wave maximum key
    int32_t my_id = -1;
    float my_l = 0.0f;
    for (int k = 0; k < K; ++k) {
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < V; ++i) best = key[i] > best ? key[i] : best;
        best = wave_max_u64(best);
        const int id = int(0xffffffffu - uint32_t(best));
#pragma unroll
        for (int i = 0; i < V; ++i)
            if (key[i] == best) key[i] = 0;
        if (lane == k) {
            my_id = id;
            my_l = l[id];
        }
    }
    // softmax pieces: max is the first selection's logit
    const float mx = __shfl(my_l, 0, 64);
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < V; ++i)
        if (64 * i + lane < E) s += double(expf(v[i] - mx));
    s = wave_sum_d(s);
    float p = 0.0f;
    if (lane < K) p = float(double(expf(my_l - mx)) / s);
    // the selected mass in rank order, as a float running sum (moe_ref.cu:158-160)
    float ws = 0.0f;
    for (int k = 0; k < K; ++k) ws += __shfl(p, k, 64);
    ws = fmaxf(ws, 6.103515625e-5f);
    if (lane < K) {
        ids[lane] = my_id;
        wts[lane] = p / ws;
        if (counts) atomicAdd(counts + my_id, 1u);
        if (tail && in_tail) atomicAdd(tail + my_id, 1u);
    }
}

// wave per token
template <int V>
__global__ void __launch_bounds__(256) k_route_topk(const float* __restrict__ logits, int T, int E, int K,
                                                    int32_t* __restrict__ ids, float* __restrict__ wts, uint32_t* counts,
                                                    uint32_t* tail, int tail_from) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    topk_wave<V>(logits + size_t(t) * E, E, K, ids + size_t(t) * K, wts + size_t(t) * K, counts, tail, t >= tail_from);
}

}  // namespace

// ---------------------------------------------------------------- host entry points

int router_logits(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                  float* logits, float* gate, hipStream_t stream) {
    if (T < 1 || E < 1 || E > kMaxE || n % 64 || n < 64 || n > 64 * 64) return set_error(kErrShape, "router: shape T=%d E=%d n=%d", T, E, n);
    if (!x || !W || !logits || (gate_w && !gate)) return set_error(kErrNull, "router: null pointer");
    const int L = n / 64;
    const int rows = E + (gate_w ? 1 : 0);
    // token tile so that the LDS tile stays within 64 KB
    int TT = int(65536 / (size_t(64) * (L + 1) * 4));
    if (TT > 16) TT = 16;
    if (TT < 1) TT = 1;
    const size_t smem = size_t(TT) * 64 * (L + 1) * 4;
    // each workgroup keeps its 8 router rows in registers over tok_per_wg tokens
    const int tok_per_wg = T <= 64 ? TT : 64;
    dim3 grid((rows + 7) / 8, (T + tok_per_wg - 1) / tok_per_wg);
#define FRT_ROUTER_L(LL)                                                                                         \
    case LL:                                                                                                     \
        k_router<LL><<<grid, 512, smem, stream>>>(x, T, W, bias, gate_w, E, logits, gate, TT, tok_per_wg);                   \
        break;
    switch (L) {
        FRT_ROUTER_L(8) FRT_ROUTER_L(16) FRT_ROUTER_L(24) FRT_ROUTER_L(32) FRT_ROUTER_L(40) FRT_ROUTER_L(48)
        FRT_ROUTER_L(56) FRT_ROUTER_L(64)
        default: return set_error(kErrShape, "router: n=%d needs n/64 in {8,16,..,64}", n);
    }
#undef FRT_ROUTER_L
    FRT_LAUNCHED("router_logits");
    return kOk;
}

int quantize_q8(const float* x, int rows, int n, int8_t* xq, float* xd, _Float16* xq16, hipStream_t stream) {
    if (rows < 1 || n % 64) return set_error(kErrShape, "quantize_q8: n=%d not a multiple of 64", n);
    const int nb = rows * (n / kQ8);
    const int waves = (nb + 1) / 2;
    k_quant_q8<<<(waves + 3) / 4, 256, 0, stream>>>(x, nb, xq, xd, xq16, n);
    FRT_LAUNCHED("quantize_q8");
    return kOk;
}

int route_topk(hipStream_t stream, const float* logits, int T, int E, int K, int32_t* ids, float* wts, uint32_t* counts,
               uint32_t* tail_counts, int tail_from) {
    if (E > kMaxE || E < 1 || K > 32 || K < 1 || K > E || T < 0) return set_error(kErrShape, "moe_route_topk: unsupported shape E=%d k=%d", E, K);
    if (T == 0) return kOk;
    if (!logits || !ids || !wts) return set_error(kErrNull, "moe_route_topk: null pointer");
    const unsigned grid = unsigned((T + 3) / 4);
    if (E <= 512) k_route_topk<8><<<grid, 256, 0, stream>>>(logits, T, E, K, ids, wts, counts, tail_counts, tail_from);
    else k_route_topk<16><<<grid, 256, 0, stream>>>(logits, T, E, K, ids, wts, counts, tail_counts, tail_from);
    FRT_LAUNCHED("moe_route_topk");
    return kOk;
}

}  // namespace frt
