/* CPU ORACLE — test infrastructure only.
 *
 * A clean-room restatement of flashrt's CPU MoE path, used as the checker for the HIP
 * library. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product path (flashrt_amd) never does.
 *
 * Every function cites the reference file:line whose semantics it restates. Parity status of
 * each function (what pins it) is listed in oracle/README.md.
 */
#ifndef FLASHRT_ORACLE_H
#define FLASHRT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- half precision (core/fp16.hpp:11-52) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- Q2_0 planar format (quant/q2_0/q2_0.hpp:5-44, q2_0.cpp:21-80) ---- */
size_t orc_mat_bytes(int rows, int cols);
size_t orc_expert_bytes(int n, int ff);
/* ggml blocks {fp16 d; u8 qs[16]} x rows*cols/64 -> planar codes then scales */
void orc_repack(const void* ggml_rows, int rows, int cols, void* dst);
/* planar code of element j (0..63) of a 16-byte block: 0..3 */
int orc_planar_code(const uint8_t* blk16, int j);

/* ---- Q8_0 activations, 32 per block (q2_0.cpp:93-117) ---- */
/* qs [n] int8; d [n/32] = fp16-rounded amax/127 as float */
void orc_quantize_q8(const float* x, int n, int8_t* qs, float* d);
void orc_quantize_q8_blk(const float* x, int n, int blk, int8_t* qs, float* d);

/* ---- matvec: y[t*ldy + r] for r in [r0,r1), t < ntok.
 * w: planar matrix (codes then scales), rows x cols. qs/d: ntok activation vectors back to back.
 * order 0: matvec_ref (q2_0.cpp:119-140, ggml generic order)
 * order 1: the AVX-512 VNNI kernel's float order (q2_0_avx512.cpp:23-52), restated in scalar code */
void orc_matvec(const uint8_t* w, int rows, int cols, const int8_t* qs, const float* d, int ntok, int r0, int r1,
                float* y, int ldy, int order);

/* ---- one expert, SwiGLU (q2_0.cpp:164-185): out[t*ldo + r], ntok <= 4 */
void orc_expert_ffn(const uint8_t* blob, int n, int ff, const int8_t* xq, const float* xd, int ntok, float* out, int ldo,
                    int order);
void orc_expert_ffn_blk(const uint8_t* blob, int n, int ff, const int8_t* xq, const float* xd, int ntok, float* out,
                        int ldo, int order, int hblk);

/* ---- router logits in the canonical order shared with the HIP kernels:
 * for each (t,e): 64 chains, chain j = fmaf over k in [j*L, (j+1)*L) ascending (L = n/64) from 0,
 * then the adjacent pairwise tree ((c0+c1)+(c2+c3))+... over the chains, then + bias[e] (bias may
 * be NULL).
 * The reference computes the logits with ggml's dense linear (blocks.hpp:85), which no reference
 * test pins; this order is this build's definition. */
void orc_router_logits(const float* x, int T, const float* W, const float* bias, int E, int n, float* logits);
float orc_dot_canon(const float* w, const float* x, int n);

/* ---- the stack's pre-MoE RMS norm in the canonical order shared with the HIP kernels:
 * ss = the same pairwise tree over 64 chains of fmaf(x, x, acc) over contiguous L = n/64 values; r = 1/sqrtf(ss/n +
 * 1e-6f); u = x * r (this build's synthetic-stack definition; the model's own norm has a weight). */
void orc_rmsnorm(const float* x, int T, int n, float* u);

/* ---- routing as moe_block's host code (arch/qwen4exp/moe_ref.cu:146-164), with the selection
 * rank defined as in test_route_topk (tests/test_route_topk.cpp:52-55): by logit descending, ties
 * to the lower expert id. counts may be NULL (else += 1 per selection). */
void orc_route_topk(const float* logits, int T, int E, int K, int32_t* ids, float* wts, uint32_t* counts);

/* ---- dispatch permutation (kernels/cuda/moe_q2.cu:83-168): a stable counting sort of the
 * slots s = t*K + k by ids[s]. bounds [E+1]; row r: slot_of[r], tok_of[r] = slot_of[r]/K. */
void orc_dispatch(const int32_t* ids, int T, int K, int E, int32_t* bounds, int32_t* tok_of, int32_t* slot_of);

/* ---- the CPU MoE (quant/q2_0/moe_cpu.cpp:36-114) over the reference's Miss list, on n_threads
 * threads (the result does not depend on it). blobs[i], ntok[i], tok[i*4+j], w[i*4+j].
 * x: Q8 activations of the window (xq [T][n], xd [T][n/32]); out [T][ldo]. */
void orc_moe_cpu(int n, int ff, const uint8_t* const* blobs, const int* ntok, const int* tok, const float* w, int n_miss,
                 const int8_t* xq, const float* xd, int T, float* out, int ldo, int n_threads, int order);

/* ---- the whole MoE layer, moe_block's semantics (arch/qwen4exp/moe_ref.cu:106-190):
 * logits (canonical router) -> routing -> misses grouped per expert (<= 4 tokens each, token
 * order, experts ascending) -> moe_cpu -> + shared expert * sigmoid(gate logit) (moe_ref.cu:90-97).
 * Routed expert e of the layer is at arena + e*stride. The shared expert is a Q2_0 blob of the
 * same shape (the BASELINE configuration's choice). Outputs: out [T][n], ids/wts [T][K].
 * norm_input: the layer runs on u = orc_rmsnorm(x) instead of x. */
void orc_moe_layer(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, const float* router_w,
                   const float* router_bias, const float* gate_w, int n, int ff, int K, const float* x, int T,
                   int n_threads, int order, float* out, int32_t* ids, float* wts, float* logits_out, int norm_input);

/* ---- the shared expert in the model's own GGUF type (moe_ref.cu:117-123 computes it with ggml's
 * linear(): ffn_gate_shexp / ffn_up_shexp [ffs][n], ffn_down_shexp [n][ffs], row-major ggml layout),
 * on the layer input x (fp32 [T][n]); out [T][n]. type (ggml ids): 0 F32, 1 F16, 30 BF16, 8 Q8_0
 * (blocks {fp16 d; int8 q[32]}). Q8_0: x and h are Q8_0 activations (orc_quantize_q8), each row
 * y = sum over blocks ascending of float(sumi) * (d_w * d_a) (ggml's vec_dot_q8_0_q8_0 order);
 * F32/F16/BF16: x and h stay fp32, y = sum_j w_j x_j with fp32 products summed in double, then
 * rounded. h = g / (1 + exp(-g)) * u (fp32). This build's definition: ggml's dense kernels are not
 * in this image, and no reference test pins the shared expert on its own. */
void orc_shexp_ffn(int type, const void* gate, const void* up, const void* down, int n, int ffs, const float* x, int T,
                   float* out);
/* one of its products: y [T][rows] = W x_t, x [T][cols] fp32 (Q8_0: quantized per token first) */
void orc_dense_mv(int type, const void* w, int rows, int cols, const float* x, int T, float* y);
/* orc_moe_layer with the shared expert given as orc_shexp_ffn's tensors (shared_type >= 0) in place of
 * a Q2_0 blob (shared_type < 0: orc_moe_layer itself). */
void orc_moe_layer_shexp(const uint8_t* arena, size_t stride, int E, int shared_type, const void* sg, const void* su,
                         const void* sd, int ffs, const uint8_t* shared_blob, const float* router_w,
                         const float* router_bias, const float* gate_w, int n, int ff, int K, const float* x, int T,
                         int n_threads, int order, float* out, int32_t* ids, float* wts, float* logits_out,
                         int norm_input);

/* ---- synthetic inputs: the seeded recipe restated independently in the HIP library ---- */
uint64_t orc_gen_key(uint64_t seed, uint64_t cfg, uint64_t layer, uint64_t tensor);
uint64_t orc_gen_u64(uint64_t key, uint64_t i);
float orc_gen_normal(uint64_t key, uint64_t i);
/* one expert blob (planar Q2_0): uniform codes, fp16(|N(0,1)|*scale_sd) scales */
void orc_gen_expert(uint64_t seed, int cfg, int layer, int expert, int n, int ff, float scale_sd, uint8_t* blob);
/* dst[i] = sd * N(0,1), i < count */
void orc_gen_normal_f32(uint64_t seed, int cfg, int layer, int tensor, float sd, float* dst, size_t count);
/* Zipf-style logit prior: bias[e] = -s * alpha * ln(1 + pi(e)), pi a seeded permutation of 0..E-1 */
void orc_gen_zipf_bias(uint64_t seed, int cfg, int layer, int E, float s, float alpha, float* bias);

#ifdef __cplusplus
}
#endif
#endif
