// The shared expert in the model's own GGUF type, and the slot path of a layer (per-slot expert
// outputs, then a combine) that it and the shapes outside the templated decode kernels take.
//
// The reference computes the shared expert with ggml's linear() on whatever type the model file
// ships (arch/qwen4exp/moe_ref.cu:117-123; moe_fast.cu:1056-1068; moe_stream.cu:169-173), then adds
// it, gated by sigmoid(ffn_gate_inp_shexp . x), in the combine (moe_fast.cu:498-542). Here:
//   - k_shexp_mv: rows of a dense ggml matrix (F32, F16, BF16 or Q8_0, row-major as in the GGUF
//     file) against a tile of TT tokens, one wave per row: gate and up together with the SwiGLU
//     (h = g / (1 + exp(-g)) * u), or the down product. Q8_0 weights take Q8_0 activations (x and
//     h quantized per 32 as the CPU path does, q8_0 . q8_0 per block as an exact integer dot, then
//     scaled by d_w d_a); the other types take the fp32 activations.
//   - the layer with such a shared expert: router logits -> route_topk -> the routed experts as
//     per-slot outputs (moe_hits for windows of up to 8 tokens, moe_q2::run for prefill chunks) ->
//     the shared expert -> k_slot_combine (the routed slots in ascending expert id, then the shared
//     expert times sigmoid(gate), then the residual: moe_cpu.cpp:63-80 and moe_ref.cu:90-97).
#include "common.hpp"
#include "../../include/flashrt_moe.h"

namespace frt {

namespace {

constexpr int kShNT = 256;   // 4 waves: one row each
constexpr int kShTT = 4;     // tokens per workgroup
constexpr int kShMaxCols = 4096;

// 32 weights of row r, block b (32 columns), as floats (dense types) -> w[32]
template <int TYPE>
__device__ __forceinline__ void dense_block(const uint8_t* row, int b, float (&w)[32]) {
    if (TYPE == FRT_GGML_F32) {
        const float4* p = reinterpret_cast<const float4*>(row) + b * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = p[i];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(row) + b * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = p[i];
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint16_t lo = uint16_t(d[k] & 0xffffu), hi = uint16_t(d[k] >> 16);
                if (TYPE == FRT_GGML_F16) {
                    w[8 * i + 2 * k] = h2f(lo);
                    w[8 * i + 2 * k + 1] = h2f(hi);
                } else {   // bf16: the upper half of an fp32
                    w[8 * i + 2 * k] = __uint_as_float(uint32_t(lo) << 16);
                    w[8 * i + 2 * k + 1] = __uint_as_float(uint32_t(hi) << 16);
                }
            }
        }
    }
}

// A pair of Q8_0 blocks 2p, 2p + 1 of a row (68 bytes from a 4-byte aligned offset): their codes as
// 8 + 8 dwords and their scales.
__device__ __forceinline__ void q8_pair(const uint8_t* row, int p, uint32_t (&q0)[8], uint32_t (&q1)[8], float& d0,
                                        float& d1) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(row + size_t(p) * 68);
    uint32_t v[17];
#pragma unroll
    for (int i = 0; i < 17; ++i) v[i] = w[i];
    d0 = h2f(uint16_t(v[0] & 0xffffu));
#pragma unroll
    for (int i = 0; i < 8; ++i) q0[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);   // bytes 2 .. 33
    d1 = h2f(uint16_t(v[8] >> 16));
#pragma unroll
    for (int i = 0; i < 8; ++i) q1[i] = v[9 + i];   // bytes 36 .. 67
}

// rows r of W1 (and W2, DUAL) against TT tokens t0 .. : out[t][r] = W1 a_t (DUAL: silu(W1 a_t) * W2 a_t).
// a: fp32 [T][cols] (dense types) or Q8_0 codes aq [T][cols] with scales ad [T][cols/32] (Q8_0).
template <int TYPE, bool DUAL>
__global__ void __launch_bounds__(kShNT) k_shexp_mv(const uint8_t* __restrict__ W1, const uint8_t* __restrict__ W2,
                                                     int rows, int cols, const float* __restrict__ af,
                                                     const int8_t* __restrict__ aq, const float* __restrict__ ad, int T,
                                                     float* __restrict__ out) {
    constexpr bool Q8 = TYPE == FRT_GGML_Q8_0;
    __shared__ __align__(16) float s_af[Q8 ? 1 : kShTT * kShMaxCols];
    __shared__ __align__(16) int8_t s_aq[Q8 ? kShTT * kShMaxCols : 16];
    __shared__ float s_ad[Q8 ? kShTT * kShMaxCols / kQ8 : 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int t0 = blockIdx.y * kShTT, tn = min(kShTT, T - t0);
    // the token tile's activations into LDS
    if (Q8) {
        const int nw = tn * cols / 4;
        for (int i = tid; i < nw; i += kShNT)
            reinterpret_cast<uint32_t*>(s_aq)[i] = reinterpret_cast<const uint32_t*>(aq + size_t(t0) * cols)[i];
        for (int i = tid; i < tn * cols / kQ8; i += kShNT) s_ad[i] = ad[size_t(t0) * (cols / kQ8) + i];
    } else {
        const int nw = tn * cols / 4;
        for (int i = tid; i < nw; i += kShNT)
            reinterpret_cast<float4*>(s_af)[i] = reinterpret_cast<const float4*>(af + size_t(t0) * cols)[i];
    }
    __syncthreads();
    const int r = blockIdx.x * 4 + wave;
    if (r >= rows) return;
    float acc1[kShTT], acc2[kShTT];
#pragma unroll
    for (int t = 0; t < kShTT; ++t) acc1[t] = acc2[t] = 0.0f;
    if (Q8) {
        const size_t rb = size_t(cols / kQ8) * 34;
        const uint8_t* row1 = W1 + size_t(r) * rb;
        const uint8_t* row2 = DUAL ? W2 + size_t(r) * rb : nullptr;
        for (int p = lane; p < cols / 64; p += 64) {
            uint32_t qa[8], qb[8];
            float da, db;
            q8_pair(row1, p, qa, qb, da, db);
            uint32_t ua[8], ub[8];
            float ea = 0.0f, eb = 0.0f;
            if (DUAL) q8_pair(row2, p, ua, ub, ea, eb);
#pragma unroll
            for (int t = 0; t < kShTT; ++t) {
                if (t >= tn) break;
                const int* xa = reinterpret_cast<const int*>(s_aq + t * cols + 64 * p);
                int s0 = 0, s1 = 0, v0 = 0, v1 = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    s0 = dot4(int(qa[i]), xa[i], s0);
                    s1 = dot4(int(qb[i]), xa[8 + i], s1);
                    if (DUAL) {
                        v0 = dot4(int(ua[i]), xa[i], v0);
                        v1 = dot4(int(ub[i]), xa[8 + i], v1);
                    }
                }
                const float x0 = s_ad[t * (cols / kQ8) + 2 * p], x1 = s_ad[t * (cols / kQ8) + 2 * p + 1];
                acc1[t] = acc1[t] + float(s0) * (da * x0);
                acc1[t] = acc1[t] + float(s1) * (db * x1);
                if (DUAL) {
                    acc2[t] = acc2[t] + float(v0) * (ea * x0);
                    acc2[t] = acc2[t] + float(v1) * (eb * x1);
                }
            }
        }
    } else {
        const size_t rb = size_t(cols) * (TYPE == FRT_GGML_F32 ? 4 : 2);
        const uint8_t* row1 = W1 + size_t(r) * rb;
        const uint8_t* row2 = DUAL ? W2 + size_t(r) * rb : nullptr;
        for (int b = lane; b < cols / 32; b += 64) {
            float w1[32], w2[32];
            dense_block<TYPE>(row1, b, w1);
            if (DUAL) dense_block<TYPE>(row2, b, w2);
#pragma unroll
            for (int t = 0; t < kShTT; ++t) {
                if (t >= tn) break;
                const float4* xp = reinterpret_cast<const float4*>(s_af + t * cols + 32 * b);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 xv = xp[i];
                    const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        acc1[t] = fmaf(w1[4 * i + k], xs[k], acc1[t]);
                        if (DUAL) acc2[t] = fmaf(w2[4 * i + k], xs[k], acc2[t]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kShTT; ++t) {
        if (t >= tn) break;
        const float g = wave_sum_tree(acc1[t]);
        if (DUAL) {
            const float u = wave_sum_tree(acc2[t]);
            if (lane == 0) out[size_t(t0 + t) * rows + r] = g / (1.0f + expf(-g)) * u;
        } else if (lane == 0) {
            out[size_t(t0 + t) * rows + r] = g;
        }
    }
}

// hit lists of moe_hits from routing ids: hit_ptr[t][k] = arena + ids[t][k] * stride for k < K, and,
// with a shared blob, hit_ptr[t][K] = shared; hit_n[t] = the slots per token (K or K + 1)
__global__ void k_hits_from_ids(const int32_t* __restrict__ ids, int T, int K, const uint8_t* arena, size_t stride,
                                const uint8_t* shared, const uint8_t** hit_ptr, int32_t* hit_n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int S = shared ? K + 1 : K;
    if (i < T * S) {
        const int t = i / S, k = i % S;
        hit_ptr[i] = k < K ? arena + size_t(ids[t * K + k]) * stride : shared;
    }
    if (i < T) hit_n[i] = S;
}

// out[t][i] = (resid) + (sum over the token's K slots in ascending expert id of w * Y[slot][i]
// + sh[t][i] * sigmoid(gate[t])). Y: per-slot rows, S slots per token, slot t * S + k in rank order
// (moe_hits' yh or moe_q2::run's yd); sh: the shared expert's row of token t at sh + t * sh_stride.
__global__ void __launch_bounds__(256) k_slot_combine(int T, int K, int S, int n, const int32_t* __restrict__ ids,
                                                      const float* __restrict__ wts, const float* __restrict__ Y,
                                                      const float* __restrict__ sh, size_t sh_stride,
                                                      const float* __restrict__ gate,
                                                      const float* __restrict__ resid, float* __restrict__ out) {
    __shared__ int s_ord[32];
    __shared__ float s_w[32];
    const int t = blockIdx.y;
    const int tid = threadIdx.x;
    if (tid < K) {   // the slot of rank r in ascending id (ids of one token are distinct)
        const int id = ids[t * K + tid];
        int r = 0;
        for (int k = 0; k < K; ++k) r += int(ids[t * K + k] < id);
        s_ord[r] = tid;
        s_w[r] = wts[t * K + tid];
    }
    __syncthreads();
    const float g = 1.0f / (1.0f + expf(-gate[t]));
    for (int i = blockIdx.x * 256 + tid; i < n; i += gridDim.x * 256) {
        float acc = 0.0f;
        for (int r = 0; r < K; ++r) {
            const float p = s_w[r] * Y[(size_t(t) * S + s_ord[r]) * n + i];
            acc = acc + p;
        }
        const float p = sh[size_t(t) * sh_stride + i] * g;
        float o = acc + p;
        if (resid) o = resid[size_t(t) * n + i] + o;
        out[size_t(t) * n + i] = o;
    }
}

}  // namespace

// ---------------------------------------------------------------- host side

bool shexp_type_ok(int type) {
    return type == FRT_GGML_F32 || type == FRT_GGML_F16 || type == FRT_GGML_BF16 || type == FRT_GGML_Q8_0;
}
bool shexp_shape_ok(int n, int ffs) {
    return n >= 64 && ffs >= 64 && n % 64 == 0 && ffs % 64 == 0 && n <= kShMaxCols && ffs <= kShMaxCols;
}

// W (rows x cols) against T tokens; DUAL: W1, W2 and the SwiGLU.
static int shexp_mv(int type, bool dual, const void* W1, const void* W2, int rows, int cols, const float* af,
                    const int8_t* aq, const float* ad, int T, float* out, hipStream_t stream) {
    const dim3 grid((rows + 3) / 4, (T + kShTT - 1) / kShTT);
    const uint8_t* w1 = static_cast<const uint8_t*>(W1);
    const uint8_t* w2 = static_cast<const uint8_t*>(W2);
#define FRT_SH(TY)                                                                                                  \
    if (dual) k_shexp_mv<TY, true><<<grid, kShNT, 0, stream>>>(w1, w2, rows, cols, af, aq, ad, T, out);             \
    else k_shexp_mv<TY, false><<<grid, kShNT, 0, stream>>>(w1, w2, rows, cols, af, aq, ad, T, out);
    switch (type) {
        case FRT_GGML_F32: FRT_SH(FRT_GGML_F32) break;
        case FRT_GGML_F16: FRT_SH(FRT_GGML_F16) break;
        case FRT_GGML_BF16: FRT_SH(FRT_GGML_BF16) break;
        case FRT_GGML_Q8_0: FRT_SH(FRT_GGML_Q8_0) break;
        default: return set_error(kErrShape, "shared expert: ggml type %d (F32, F16, BF16 or Q8_0)", type);
    }
#undef FRT_SH
    FRT_LAUNCHED("shared expert");
    return kOk;
}

int quantize_q8(const float* x, int rows, int n, int8_t* xq, float* xd, _Float16* xhi, _Float16* xlo,
                hipStream_t stream);

size_t shexp_ws_bytes(int T, int n, int ffs) {
    return up256(size_t(T) * ffs * 4) + up256(size_t(T) * ffs) + up256(size_t(T) * (ffs / kQ8) * 4);
}

// sh [T][n] = the shared expert of type `type` on u [T][n]; uq/ud: u's Q8_0 (Q8_0 type only; may be
// null, then computed into the workspace's h area first... the caller passes them). ws: shexp_ws_bytes.
int shexp_run(int type, const void* g, const void* u, const void* d, int n, int ffs, const float* x, const int8_t* xq,
              const float* xd, int T, float* sh, void* ws, hipStream_t stream) {
    if (!shexp_type_ok(type)) return set_error(kErrShape, "shared expert: ggml type %d (F32, F16, BF16 or Q8_0)", type);
    if (!shexp_shape_ok(n, ffs)) return set_error(kErrShape, "shared expert: n=%d ffs=%d", n, ffs);
    uint8_t* p = static_cast<uint8_t*>(ws);
    float* h = reinterpret_cast<float*>(p);
    p += up256(size_t(T) * ffs * 4);
    int8_t* hq = reinterpret_cast<int8_t*>(p);
    p += up256(size_t(T) * ffs);
    float* hd = reinterpret_cast<float*>(p);
    if (type == FRT_GGML_Q8_0) {
        if (int rc = shexp_mv(type, true, g, u, ffs, n, nullptr, xq, xd, T, h, stream)) return rc;
        if (int rc = quantize_q8(h, T, ffs, hq, hd, nullptr, nullptr, stream)) return rc;
        return shexp_mv(type, false, d, nullptr, n, ffs, nullptr, hq, hd, T, sh, stream);
    }
    if (int rc = shexp_mv(type, true, g, u, ffs, n, x, nullptr, nullptr, T, h, stream)) return rc;
    return shexp_mv(type, false, d, nullptr, n, ffs, h, nullptr, nullptr, T, sh, stream);
}

int hits_from_ids(const int32_t* ids, int T, int K, const uint8_t* arena, size_t stride, const uint8_t* shared,
                  const uint8_t** hit_ptr, int32_t* hit_n, hipStream_t stream) {
    const int cnt = T * (K + 1);
    k_hits_from_ids<<<(cnt + 255) / 256, 256, 0, stream>>>(ids, T, K, arena, stride, shared, hit_ptr, hit_n);
    FRT_LAUNCHED("hit lists");
    return kOk;
}

int slot_combine(int T, int K, int S, int n, const int32_t* ids, const float* wts, const float* Y, const float* sh,
                 size_t sh_stride, const float* gate, const float* resid, float* out, hipStream_t stream) {
    if (K < 1 || K > 32) return set_error(kErrShape, "combine: K=%d", K);
    const dim3 grid((n + 255) / 256 < 8 ? (n + 255) / 256 : 8, T);
    k_slot_combine<<<grid, 256, 0, stream>>>(T, K, S, n, ids, wts, Y, sh, sh_stride, gate, resid, out);
    FRT_LAUNCHED("combine");
    return kOk;
}

}  // namespace frt
