// C++ mirror of flashrt's MoE-path call surface over the C ABI of libflashrt_moe.so
// (include/flashrt_moe.h). Header-only; link with -lflashrt_moe.
//
// Names, argument order and error behaviour follow the reference's C++ entry points, with
// cudaStream_t replaced by hipStream_t:
//   flashrt::ExpertArena / arena_alloc / arena_free   core/expert_arena.hpp:14-30
//   flashrt::qwen4exp::moe_route_topk                 arch/qwen4exp/blocks.hpp:130-135
//   flashrt::moe_q2::workspace_bytes / run            kernels/cuda/moe_q2.h:20-30
//   flashrt::qwen4exp::moe_hits_scratch_bytes / moe_hits   arch/qwen4exp/moe_fast.hpp:134-142
//   flashrt::qwen4exp::MoeLayer::forward              moe_block_fast / moe_block_stream /
//                                                     moe_block (moe_fast.hpp:144-147,
//                                                     moe_stream.hpp:35, blocks.hpp:286)
// A nonzero status from the library becomes std::runtime_error carrying frt_last_error(), where
// the reference throws std::runtime_error. Every call only enqueues on the given stream.
//
// The arena lives in device memory (HBM) rather than pinned host RAM: arena_alloc's PageMode and
// touch_threads are accepted for source compatibility and ignored.
#ifndef FLASHRT_MOE_HPP
#define FLASHRT_MOE_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "flashrt_moe.h"

namespace flashrt {

namespace detail {
inline void check(int rc, const char* what) {
    if (rc != FRT_OK) throw std::runtime_error(std::string(what) + ": " + frt_last_error());
}
}  // namespace detail

// core/platform.hpp's page modes; the device arena has no host pages, so the mode is ignored.
enum class PageMode { Default, Huge, Pinned };

struct ExpertArena {
    frt_arena raw{};
    size_t blob_bytes = 0;   // useful bytes per expert
    size_t stride = 0;       // blob_bytes rounded up to 4 KiB
    int n_layer = 0, n_expert = 0;

    uint8_t* blob(int layer, int expert) const { return frt_arena_blob(&raw, layer, expert); }
    size_t total_bytes() const { return frt_arena_total_bytes(&raw); }
    uint8_t* base() const { return raw.base; }
};

// Returns an arena with base() == nullptr on failure, as the reference's does.
inline ExpertArena arena_alloc(int n_layer, int n_expert, size_t blob_bytes, PageMode = PageMode::Default,
                               int /*touch_threads*/ = 0) {
    ExpertArena a;
    if (frt_arena_alloc(n_layer, n_expert, blob_bytes, &a.raw) != FRT_OK) return ExpertArena{};
    a.blob_bytes = a.raw.blob_bytes;
    a.stride = a.raw.stride;
    a.n_layer = a.raw.n_layer;
    a.n_expert = a.raw.n_expert;
    return a;
}

inline void arena_free(ExpertArena& a) {
    if (a.raw.base) frt_arena_free(&a.raw);
    a = ExpertArena{};
}

// Copies one planar host blob into (layer, expert) on `stream` (the loader's last step,
// arch/qwen4exp/experts.cpp:113-115, with the arena in HBM).
inline void arena_upload(const ExpertArena& a, int layer, int expert, const void* host_blob, hipStream_t stream) {
    detail::check(frt_arena_upload(&a.raw, layer, expert, host_blob, stream), "arena_upload");
}

namespace q2_0 {
inline size_t mat_bytes(int rows, int cols) { return frt_q2_mat_bytes(rows, cols); }
inline size_t expert_bytes(int d_model, int d_ff) { return frt_q2_expert_bytes(d_model, d_ff); }
}  // namespace q2_0

namespace qwen4exp {

inline void moe_route_topk(hipStream_t stream, const float* logits, int T, int E, int k, int32_t* ids, float* wts,
                           uint32_t* counts, uint32_t* tail_counts = nullptr, int tail_from = 1 << 30) {
    detail::check(frt_moe_route_topk(stream, logits, T, E, k, ids, wts, counts, tail_counts, tail_from),
                  "moe_route_topk");
}

// The reference sizes the scratch without d_model; this library also keeps the window's Q8
// activations there, so the size takes d_model (default: the largest supported, 16384).
inline size_t moe_hits_scratch_bytes(int K, int ff, int T = 1, int d_model = 16384) {
    return frt_moe_hits_scratch_bytes(K, ff, T, d_model);
}

inline void moe_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const float* x, int n, int ff,
                     void* scratch, float* yh, hipStream_t stream, int T = 1) {
    detail::check(frt_moe_hits(hit_ptr, hit_n, K, x, n, ff, scratch, yh, stream, T), "moe_hits");
}

// One MoE layer on the HBM arena (router -> top-k -> routed experts + gated shared expert).
struct MoeLayer {
    frt_moe_layer desc{};

    MoeLayer(const uint8_t* experts, size_t stride, int n_expert, const uint8_t* shared, const float* router_w,
             const float* router_bias, const float* gate_w, int d_model, int d_ff, int top_k, bool norm_input = false) {
        desc = frt_moe_layer{experts, stride, n_expert, shared, router_w, router_bias, gate_w,
                             d_model, d_ff,   top_k,    norm_input ? FRT_LAYER_NORM_INPUT : 0};
    }
    size_t workspace_bytes(int T) const { return frt_moe_layer_workspace_bytes(&desc, T); }
    // out [T][d_model] = (resid ? resid : 0) + moe(x); ids/wts [T][top_k], counts [E] optional.
    void forward(const float* x, int T, float* out, void* ws, size_t ws_bytes, hipStream_t stream,
                 const float* resid = nullptr, int32_t* ids = nullptr, float* wts = nullptr,
                 uint32_t* counts = nullptr) const {
        detail::check(frt_moe_layer_forward(&desc, x, T, resid, out, ids, wts, counts, ws, ws_bytes, stream),
                      "moe_layer_forward");
    }
};

}  // namespace qwen4exp

namespace moe_q2 {

inline size_t workspace_bytes(int T, int K, int n, int ff, int E) { return frt_moe_q2_workspace_bytes(T, K, n, ff, E); }

inline void run(const uint8_t* experts, size_t stride, int E, int n, int ff, const float* x, const int32_t* ids, int T,
                int K, void* yd, void* ws, size_t ws_bytes, hipStream_t stream, bool block64 = false,
                bool yd_bf16 = false) {
    detail::check(frt_moe_q2_run(experts, stride, E, n, ff, x, ids, T, K, yd, ws, ws_bytes, stream, block64 ? 1 : 0,
                                 yd_bf16 ? 1 : 0),
                  "moe_q2::run");
}

}  // namespace moe_q2
}  // namespace flashrt

#endif
