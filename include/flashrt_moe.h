/* flashrt_moe.h — C ABI of the MI355X (gfx950) MoE-layer library, libflashrt_moe.so.
 *
 * Each entry point replaces one entry of the reference's C++ MoE call surface; the reference
 * declaration it stands for is cited beside it (paths into BFinn/flashrt). Conventions kept from
 * the reference:
 *   - every device buffer and workspace is allocated by the caller; each kernel family has a
 *     *_bytes() size query; no call allocates device memory (graph capture stays legal);
 *   - calls only enqueue work on the given stream (no host synchronisation);
 *   - layouts: token-major [T][n] fp32 activations, ids/wts [T][K], per-slot outputs [T*K][n],
 *     expert blobs in the planar Q2_0 layout (quant/q2_0/q2_0.hpp:5-15): gate [ff][n] | up [ff][n] |
 *     down [n][ff], each as codes [rows][cols/64][16] then fp16 scales [rows][cols/64].
 * Errors: functions return 0 on success and a negative FRT_ERR_* code otherwise (the reference
 * throws std::runtime_error in the same places); frt_last_error() gives the message.
 * All pointers are device pointers unless stated. hipStream_t is passed as void*.
 */
#ifndef FLASHRT_MOE_H
#define FLASHRT_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FRT_OK 0
#define FRT_ERR_SHAPE -1      /* unsupported shape or argument */
#define FRT_ERR_WORKSPACE -2  /* workspace or scratch too small */
#define FRT_ERR_HIP -3        /* a HIP call failed */
#define FRT_ERR_NULL -4       /* a required pointer is missing */
#define FRT_ERR_IO -5         /* a file could not be opened or read */
#define FRT_ERR_SYNC -6       /* an earlier persistent decode call on this device ran out of time waiting
                                 for another workgroup (its outputs are undefined); reported once, by the
                                 next layer or stack call, which then launches nothing */

/* Message of the last failure on this thread (static storage; "" when none). */
const char* frt_last_error(void);
/* Library version string. */
const char* frt_version(void);

/* Per-kernel timing for measurement harnesses (no reference counterpart; the reference times
 * kernels with CUDA events in its tests, tests/test_moe_hits.cpp:183-208). Between begin and end,
 * each library call records a hipEvent on its stream after every kernel it launches; end
 * synchronises and writes, per kernel name, the summed milliseconds and launch count (names in
 * rows of name_len bytes). Returns the number of names. Do not use under graph capture. */
void frt_timing_begin(void);
int frt_timing_end(char* names, int name_len, double* total_ms, int* launches, int max);

/* ---- planar Q2_0 sizes (quant/q2_0/q2_0.hpp:40,51: mat_bytes, expert_bytes) ---- */
size_t frt_q2_mat_bytes(int rows, int cols);
size_t frt_q2_expert_bytes(int d_model, int d_ff);

/* ---- HBM expert arena (core/expert_arena.hpp:14-30: ExpertArena, arena_alloc, arena_free).
 * One device allocation of n_layer * n_expert blobs, each at a 4 KiB-aligned stride; expert e of
 * layer l is at base + (l * n_expert + e) * stride. The reference's arena lives in host RAM and
 * is registered for DMA (arch/qwen4exp/moe_fast.hpp:109-112 arena_register); on MI355X all experts
 * are resident in HBM, so this one allocation at load time replaces both. */
typedef struct frt_arena {
    uint8_t* base;      /* device */
    size_t blob_bytes;  /* useful bytes per expert */
    size_t stride;      /* blob_bytes rounded up to 4 KiB */
    int n_layer, n_expert;
} frt_arena;
int frt_arena_alloc(int n_layer, int n_expert, size_t blob_bytes, frt_arena* out);
int frt_arena_free(frt_arena* a);
uint8_t* frt_arena_blob(const frt_arena* a, int layer, int expert);
size_t frt_arena_total_bytes(const frt_arena* a);
/* ---- Q2_0 repack, ggml block order -> planar (quant/q2_0/q2_0.cpp:21-62 repack, :64-80 repack_expert),
 * host memory. A ggml block is {fp16 d; u8 qs[16]}, element j at byte j/4, bits 2(j%4). frt_q2_repack
 * writes mat_bytes(rows, cols) bytes and returns that count (0 on a bad shape: cols a multiple of 64). */
size_t frt_q2_repack(const void* ggml_rows, int rows, int cols, void* dst);
int frt_q2_repack_expert(const void* gate, const void* up, const void* down, int d_model, int d_ff, void* blob);

/* ---- expert loader (arch/qwen4exp/experts.cpp:65-131 load_experts): the three expert slabs of every
 * layer (ffn_gate_exps, ffn_up_exps, ffn_down_exps: n_expert consecutive ggml-layout Q2_0 matrices,
 * gate/up [d_ff][d_model], down [d_model][d_ff]) read with O_DIRECT from GGUF shard files, repacked
 * and uploaded into the HBM arena (one copy per 32 experts). slabs [n_layer][3] give each slab's
 * shard and absolute file offset (GgufTensor::shard / file_offset). Synchronous; FRT_ERR_IO on a
 * failed open or read. */
typedef struct frt_expert_slab {
    int shard;
    uint64_t file_offset;
} frt_expert_slab;
typedef struct frt_load_stats {
    double seconds;
    uint64_t bytes_read;
} frt_load_stats;
int frt_load_experts(const char* const* shards, int n_shards, const frt_expert_slab* slabs, int d_model, int d_ff,
                     const frt_arena* arena, int threads, frt_load_stats* stats);

/* Copies one repacked blob from host memory into (layer, expert) (the per-expert step of
 * arch/qwen4exp/experts.cpp:93-116 load_experts, minus the file read). */
int frt_arena_upload(const frt_arena* a, int layer, int expert, const void* host_blob, void* stream);

/* ---- routing (arch/qwen4exp/blocks.hpp:130-135 moe_route_topk): softmax over E <= 1024 logits,
 * top-k (k <= 32) ranked by logit, ties to the lower expert id, weights p / max(sum_top p, 2^-14);
 * counts [E] (optional) += 1 per selection; tail_counts likewise for tokens t >= tail_from. */
int frt_moe_route_topk(void* stream, const float* logits, int T, int E, int k, int32_t* ids, float* wts,
                       uint32_t* counts, uint32_t* tail_counts, int tail_from);

/* ---- router logits in the canonical order (the reference computes them with its dense linear(),
 * arch/qwen4exp/blocks.hpp:85, ffn_gate_inp and ffn_gate_inp_shexp; this build fixes one float
 * order so CPU and GPU agree bit for bit): logits [T][E] = W x + bias (bias optional), and, when
 * gate_w is given, gate [T] = gate_w . x. n a multiple of 512 up to 4096. */
int frt_router_logits(void* stream, const float* x, int T, const float* W, const float* bias, const float* gate_w,
                      int E, int n, float* logits, float* gate);

/* ---- the same router logits for many tokens (a prefill chunk) as a K-split GEMM on the matrix
 * cores, bit for bit the canonical order of frt_router_logits. n a multiple of 512 up to 4096;
 * ws of frt_router_gemm_workspace_bytes(T, E, gate_w != NULL). */
size_t frt_router_gemm_workspace_bytes(int T, int E, int has_gate);
int frt_router_logits_gemm(void* stream, const float* x, int T, const float* W, const float* bias, const float* gate_w,
                           int E, int n, float* logits, float* gate, void* ws, size_t ws_bytes);

/* ---- router / gate tensors in the model's GGUF types, widened to the fp32 layout the router
 * kernels take (the reference reads ffn_gate_inp and ffn_gate_inp_shexp through ggml's linear(),
 * arch/qwen4exp/blocks.hpp:85, in whatever type the file ships). type is the ggml type id:
 * FRT_GGML_F32 (copy), FRT_GGML_F16, FRT_GGML_BF16 or FRT_GGML_Q8_0 (blocks {fp16 d; int8 q[32]},
 * value d * q). Every one widens to fp32 exactly, so the router's canonical order then runs on the
 * model's own values. count values (a multiple of 32 for Q8_0); src and dst device pointers. */
#define FRT_GGML_F32 0
#define FRT_GGML_F16 1
#define FRT_GGML_Q8_0 8
#define FRT_GGML_BF16 30
int frt_router_widen(void* stream, const void* src, int type, size_t count, float* dst);

/* ---- Q8_0 activation quantization (quant/q2_0/q2_0.hpp:66-70 quantize_q8): per 32 values
 * d = fp16(amax/127), q = roundf(x * 127/amax). xq [rows][n] int8, xd [rows][n/32] float. */
int frt_quantize_q8(void* stream, const float* x, int rows, int n, int8_t* xq, float* xd);

/* ---- the prefill GEMMs' activation operand. No counterpart in the reference (its moe_q2 keeps int8
 * codes, moe_q2.cu:58-81); exposed so that the format can be checked on its own. Per row: the Q8_0
 * values a = q * d (blocks of `block` = 32 or 64 values, as frt_quantize_q8 / moe_q2's block64)
 * as exact fp16 pairs hi = fp16(a), lo = fp16(a - hi), in rows of np = n rounded up to 512; value k
 * of each 256-wide stretch sits at position perm256(k) of it (the order the GEMM's lanes load),
 * the pad (k >= n) is zero. n a multiple of 128. xhi / xlo [rows][np] fp16. */
int frt_quantize_pairs(void* stream, const float* x, int rows, int n, int block, uint16_t* xhi, uint16_t* xlo);

/* ---- dispatch permutation (kernels/cuda/moe_q2.cu:83-168): a stable sort of slots s = t*K + k by
 * ids[s]: bounds [E+1], row r holds slot_of[r] and tok_of[r] = slot_of[r] / K. */
size_t frt_moe_dispatch_workspace_bytes(int T, int K, int E);
int frt_moe_dispatch(void* stream, const int32_t* ids, int T, int K, int E, int32_t* bounds, int32_t* tok_of,
                     int32_t* slot_of, void* ws, size_t ws_bytes);

/* ---- prefill grouped expert GEMM (kernels/cuda/moe_q2.h:20-30 moe_q2::workspace_bytes, run).
 * yd [T*K][n]: slot t*K + k gets down(silu(gate x_t) * up x_t) of expert ids[t*K + k], expert e's
 * blob at experts + e * stride. yd_bf16 selects bf16 output. block64: x and h are quantized in Q8
 * blocks of 64 values instead of the CPU path's 32 (moe_q2.cu's AB = 64). Shapes: n and ff multiples
 * of 128 (moe_q2.cu:516-517), ff at most 4096; ff above 1024 takes fp32 yd only (the down GEMM adds
 * up chunks of 1024 in it). FRT_ERR_SHAPE otherwise. */
size_t frt_moe_q2_workspace_bytes(int T, int K, int n, int ff, int E);
int frt_moe_q2_run(const uint8_t* experts, size_t stride, int E, int n, int ff, const float* x, const int32_t* ids,
                   int T, int K, void* yd, void* ws, size_t ws_bytes, void* stream, int block64, int yd_bf16);

/* ---- decode expert GEMVs (arch/qwen4exp/moe_fast.hpp:134-142 moe_hits_scratch_bytes, moe_hits).
 * yh [T][K][n]: entry (t, k) for k < hit_n[t] = down(silu(gate x) * up x) of the blob at
 * hit_ptr[t*K + k] (device array of device pointers); entries k >= hit_n[t] are not written.
 * Shapes: n a multiple of 512 (up to 16384), ff a multiple of 64 up to 4096 (moe_fast.cu:557).
 * x [T][n] fp32, any T >= 1: one launch takes up to 8 tokens (the reference's kMaxWindow,
 * moe_fast.cu:38) and 128 (token, slot) items, and reads each distinct blob once per four of its
 * tokens (moe_fast.cu:195-355); a longer window runs in such launches, one after the other.
 * Activations are quantized to Q8_0 per 32 (the reference quantizes per 64 here); the scratch holds
 * them for any n the call takes (so its size needs no n, as the reference's). */
size_t frt_moe_hits_scratch_bytes(int K, int ff, int T);
int frt_moe_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const float* x, int n, int ff,
                 void* scratch, float* yh, void* stream, int T);

/* ---- one whole MoE layer on an HBM-resident arena: router logits -> route_topk -> routed experts
 * + shared expert * sigmoid(gate) (moe_block_fast, arch/qwen4exp/moe_fast.hpp:144-147, for T <= 8:
 * T = 1 as one persistent launch, 2..8 through the moe_hits kernels;
 * moe_block_stream, arch/qwen4exp/moe_stream.hpp:35, for prefill chunks; same math as moe_block,
 * arch/qwen4exp/blocks.hpp:286). out [T][n] = (resid ? resid : 0) + moe(u), with u = x, or with
 * flags & FRT_LAYER_NORM_INPUT u = x / rms(x) (the unweighted RMS norm that precedes the MoE in the
 * model, r = 1/sqrt(sum(x^2)/n + 1e-6) summed in the router's canonical order). ids/wts [T][K]
 * (optional outputs), counts [E] optional. */
#define FRT_LAYER_NORM_INPUT 1
typedef struct frt_moe_layer {
    const uint8_t* experts;   /* routed expert 0 of this layer; expert e at experts + e * stride */
    size_t stride;
    int n_expert;             /* E <= 1024 */
    const uint8_t* shared;    /* the shared expert's planar Q2_0 blob (same shape) */
    const float* router_w;    /* [E][n] fp32 (ffn_gate_inp) */
    const float* router_bias; /* [E] added to the logits, or NULL */
    const float* gate_w;      /* [n] fp32 (ffn_gate_inp_shexp) */
    int d_model, d_ff, top_k;
    int flags;                /* FRT_LAYER_* */
    /* Optional (NULL: none): the router matrix [E][n] the NEXT layer call will read. A decode call
     * loads it into the GPU's caches during its last kernel, each 2-row slice on the XCD whose L2
     * the next router kernel reads it from, so that the next router kernel does not wait on HBM.
     * No reference counterpart (the reference's router is a ggml linear, blocks.hpp:85). */
    const float* next_router_w;
    /* Optional: the shared expert as the model's dense GGUF tensors (ffn_gate_shexp, ffn_up_shexp
     * [shared_ff][d_model], ffn_down_shexp [d_model][shared_ff], ggml row-major layout, device memory)
     * instead of the planar Q2_0 blob `shared` (arch/qwen4exp/moe_ref.cu:117-123 computes it with
     * linear() in whatever type the file ships). shared_dense = 0 (the default): `shared` is used.
     * shared_type: FRT_GGML_F32, FRT_GGML_F16, FRT_GGML_BF16 or FRT_GGML_Q8_0 (Q8_0 weights take the
     * input and h as Q8_0 activations, per-block integer dots; the others fp32 activations).
     * shared_ff a multiple of 64, at most 4096. Such a layer runs router -> route_topk -> the routed
     * experts as per-slot outputs (moe_hits up to 8 tokens, moe_q2::run beyond) -> the shared expert
     * -> the combine; the persistent single-token kernels take only the Q2_0 blob. */
    int shared_dense;
    int shared_type;
    int shared_ff;
    const void* shared_gate;
    const void* shared_up;
    const void* shared_down;
} frt_moe_layer;
/* frt_moe_layer_forward with the routing records of moe_route_topk and MoeTrace (blocks.hpp:130-135,
 * :267-286): tail_counts [E] (optional) += 1 per selection of tokens t >= tail_from; probs [T][K]
 * (optional) = each selection's probability before renormalisation, exp(l - max) / sum_e exp(l_e - max)
 * (the sum in double, as moe_block). */
int frt_moe_layer_forward_ex(const frt_moe_layer* L, const float* x, int T, const float* resid, float* out,
                             int32_t* ids, float* wts, uint32_t* counts, uint32_t* tail_counts, int tail_from,
                             float* probs, void* ws, size_t ws_bytes, void* stream);
/* The workspace's first bytes hold the single-token path's synchronisation words: they are zeroed by
 * the first call that sees a workspace address and must not be written by the caller between calls.
 * A workspace newly allocated at an address used before (a caching allocator hands freed memory out
 * again) must be zeroed by the caller before its first call: its leftover bytes could by chance carry
 * a word the next call waits for. The size depends only on the shapes and T, not on frt_set_option. */
size_t frt_moe_layer_workspace_bytes(const frt_moe_layer* L, int T);
int frt_moe_layer_forward(const frt_moe_layer* L, const float* x, int T, const float* resid, float* out, int32_t* ids,
                          float* wts, uint32_t* counts, void* ws, size_t ws_bytes, void* stream);

/* Runtime options (no reference counterpart; for tests and measurement harnesses):
 *   "decode_fused" (default 1): single-token layer calls run as one persistent launch (router, then
 *       routing + gate/up, then down, joined inside the kernel); 0 selects the three-kernel path
 *       (router kernel, routing + gate/up kernel, down kernel). Both give identical results.
 *   "decode_xcd" (default 0): 1 runs persistent single-token calls in the kernel that splits each layer
 *       by XCD (router logits relayed into each XCD's L2, each XCD a share of the experts' ff rows,
 *       XCD partials summed last) where the shape fits; outputs within the layer bar of the default
 *       kernel's, not bit-equal to them.
 *   "decode_window_persistent" (default 1): decode windows of 2-4 tokens run as one persistent launch
 *       (routing, gate/up and down joined inside the kernel) where the shape fits; 0 selects the
 *       four-launch window path. Both give identical results.
 *   "decode_stamps" (default 0): a device buffer of 64 x 12 x 1024 uint64 that the XCD-split kernel
 *       fills with per-layer phase times, and the persistent window kernel with its 10 phase times
 *       per workgroup (100 MHz ticks; measurement only), or 0 for none.
 *   "decode_grid" (default 0): workgroups of a persistent single-token call, at most one per CU (0:
 *       one per CU).
 *   "sync_ticks" (default 20000000): bound of a persistent call's waits for other workgroups, in
 *       ticks of the GPU's 100 MHz constant clock; past it the call completes with undefined
 *       outputs and sets the error word that frt_moe_layer_sync_error reports.
 * Returns FRT_ERR_SHAPE for an unknown name or a bad value. Not thread-safe against running calls. */
int frt_set_option(const char* name, int64_t value);
/* Reads and clears the error word of a layer workspace (synchronises the stream): 1 if a persistent
 * single-token call on this workspace ran out of time waiting for another workgroup since the last
 * check, 0 if not, negative on a HIP error. Also clears the device's pending FRT_ERR_SYNC. Without this
 * call, the next frt_moe_layer_forward(_ex) / frt_moe_stack_forward on the device returns FRT_ERR_SYNC
 * (no synchronisation needed: the kernel sets a flag in pinned host memory). No reference counterpart. */
int frt_moe_layer_sync_error(void* ws, void* stream);

/* ---- allocation-free decode: frt_moe_layer_forward for decode windows (1 <= T <= 4, T * K <= 63)
 * with the workspace taken from a static device array of frt_noalloc_scratch_bytes() (4 MiB) per
 * GPU, held until the process ends. No reference counterpart: for callers that cannot allocate
 * device memory or pass a workspace (code under graph capture, tight serving loops, harnesses that
 * forbid allocation). The call itself allocates nothing. All calls on one GPU share that GPU's
 * array: calls that overlap on one GPU (other streams, other host threads) race. Larger T, or a
 * shape whose workspace exceeds the array, is refused (FRT_ERR_SHAPE / FRT_ERR_WORKSPACE). */
size_t frt_noalloc_scratch_bytes(void);
int frt_moe_layer_forward_noalloc(const frt_moe_layer* L, const float* x, int T, const float* resid, float* out,
                                  int32_t* ids, float* wts, uint32_t* counts, void* stream);
/* frt_moe_layer_sync_error for the static array of the current device (synchronises the stream): 1 if
 * an allocation-free single-token call ran out of time waiting for another workgroup since the last
 * check, else 0. No reference counterpart; for the same callers as frt_moe_layer_forward_noalloc. */
int frt_noalloc_sync_error(void* stream);

/* ---- a stack of single-token MoE layers (no reference counterpart as one call: the engine calls
 * moe_block_fast once per layer, arch/qwen4exp/forward.cu:214-217; BASELINE config 2 is a stack of
 * MoE layers chained by the residual). x_0 = x, x_{l+1} = x_l + moe_l(x_l) with each layer's own
 * flags (all layers share E, K, d_model, d_ff, stride and flags), out = x_{n_layer} [d_model].
 * ids/wts [n_layer][K] optional. Runs as one persistent launch per 64 layers ("decode_fused", the
 * default), else as n_layer calls of frt_moe_layer_forward; both give identical results. The last
 * layer's next_router_w (if any) is warmed for the next call. */
size_t frt_moe_stack_workspace_bytes(const frt_moe_layer* layers, int n_layer);
int frt_moe_stack_forward(const frt_moe_layer* layers, int n_layer, const float* x, float* out, int32_t* ids,
                          float* wts, void* ws, size_t ws_bytes, void* stream);

/* ---- seeded synthetic inputs written on the device (no reference counterpart: the reference's
 * tests draw from std::mt19937; this recipe is documented in flashrt_amd/csrc/gen.hip) ---- */
int frt_gen_experts(uint64_t seed, int cfg, int layer, int e0, int count, int tensor_base, int n, int ff, float sd,
                    uint8_t* dst, size_t stride, void* stream);
int frt_gen_normal(uint64_t seed, int cfg, int layer, int tensor, float sd, float* dst, size_t count, int round_bf16,
                   void* stream);
int frt_gen_correlated(uint64_t seed, int cfg, int layer, int tensor0, int T, int n, float rho, float* dst, void* stream);
void frt_gen_zipf_bias(uint64_t seed, int cfg, int layer, int E, float s, float alpha, float* host_bias);

#ifdef __cplusplus
}
#endif
#endif
