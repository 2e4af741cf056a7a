// C++ mirror of flashrt's MoE-path call surface over the C ABI of libflashrt_moe.so
// (include/flashrt_moe.h). Header-only; link with -lflashrt_moe.
//
// Names, argument order, types the call sites touch, and error behaviour follow the reference's
// C++ entry points, with cudaStream_t replaced by hipStream_t, so that its call sites compile as
// they are (engine/session.cpp:113-117,171-179,375-381; tools/fr_bench.cpp:204-213,403-423;
// arch/qwen4exp/forward.cu:214-217):
//   flashrt::PageMode / ExpertArena / arena_alloc / arena_free   core/platform.hpp:12-27, core/expert_arena.hpp:14-30
//   flashrt::q2_0::ExpertShape / mat_bytes / expert_bytes /
//                  repack / repack_expert                         quant/q2_0/q2_0.hpp:27-60
//   flashrt::qwen4exp::load_experts / LoadStats                   arch/qwen4exp/experts.hpp:16-25
//   flashrt::qwen4exp::arena_register                              arch/qwen4exp/moe_fast.hpp:109-112
//   flashrt::qwen4exp::moe_route_topk                              arch/qwen4exp/blocks.hpp:130-135
//   flashrt::moe_q2::workspace_bytes / run                         kernels/cuda/moe_q2.h:20-30
//   flashrt::qwen4exp::moe_hits_scratch_bytes / moe_hits           arch/qwen4exp/moe_fast.hpp:134-142
//   flashrt::qwen4exp::ExpertCache / alloc_expert_cache / expert_cache_fill / MoeFastHost /
//     alloc_moe_fast_host / start_doorbell / doorbell_* / CachePolicyConfig / create_cache_manager /
//     cache_manager_step / cache_manager_stats / cache_check / enable_pcie_misses
//                                                                  arch/qwen4exp/moe_fast.hpp:16-132
//   flashrt::qwen4exp::moe_block_fast                              arch/qwen4exp/moe_fast.hpp:144-147
//   flashrt::qwen4exp::ExpertStream / create_expert_stream / expert_stream_prefetch /
//     moe_block_stream / expert_stream_bytes(_for) / destroy_expert_stream
//                                                                  arch/qwen4exp/moe_stream.hpp:18-36
//   flashrt::qwen4exp::MoeLayer (one layer; forward(), trace)      moe_block (blocks.hpp:267-286)
// A nonzero status from the library becomes std::runtime_error carrying frt_last_error(), where the
// reference throws std::runtime_error. Every call only enqueues on the given stream, except the
// loader and the set-up calls, which are synchronous as in the reference.
//
// What differs by design: every expert is resident in HBM (288 GB per MI355X). The arena is one
// device allocation (its PageMode and touch threads are accepted and ignored); the expert cache is
// the arena itself (table[l][e] = l * n_expert + e, slot bytes = the arena stride, every lookup a
// hit), so the cache fill, the cache manager, the doorbell and the PCIe-miss set-up have nothing to
// do. The engine types these calls take (Spec, Gguf, BlockCtx, CpuPool) stay the engine's: the
// entry points that take them are templates over them and read only the members the reference's
// own calls read (Spec: n_layer, n_expert, d_model, d_ff_expert; Gguf: shards, tensor(name) ->
// shard, file_offset; BlockCtx: stream). The per-layer weights a layer call needs (router, shared
// expert, gate) are registered once per layer with set_layer() on the MoeFastHost / ExpertStream.
#ifndef FLASHRT_MOE_HPP
#define FLASHRT_MOE_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "flashrt_moe.h"

namespace flashrt {

namespace detail {
inline void check(int rc, const char* what) {
    if (rc != FRT_OK) throw std::runtime_error(std::string(what) + ": " + frt_last_error());
}
inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace detail

// core/platform.hpp's page modes (the device arena has no host pages: accepted and ignored)
enum class PageMode {
    Default,
    THP,
    HugeTLB,
};

// The arena's one allocation (the reference's HostBuffer: ptr, bytes, mode), here device memory.
struct ArenaBuffer {
    void* ptr = nullptr;
    std::size_t bytes = 0;
    PageMode mode = PageMode::Default;
};

struct ExpertArena {
    ArenaBuffer buf;
    size_t blob_bytes = 0;   // useful bytes per expert
    size_t stride = 0;       // blob_bytes rounded up to 4 KiB
    int n_layer = 0, n_expert = 0;

    uint8_t* blob(int layer, int expert) const {
        return static_cast<uint8_t*>(buf.ptr) + (size_t(layer) * n_expert + expert) * stride;
    }
    size_t total_bytes() const { return size_t(n_layer) * n_expert * stride; }
    frt_arena raw() const { return frt_arena{static_cast<uint8_t*>(buf.ptr), blob_bytes, stride, n_layer, n_expert}; }
};

// Returns an arena with buf.ptr == nullptr on failure, as the reference's does.
inline ExpertArena arena_alloc(int n_layer, int n_expert, size_t blob_bytes, PageMode mode, int /*touch_threads*/) {
    frt_arena r{};
    if (frt_arena_alloc(n_layer, n_expert, blob_bytes, &r) != FRT_OK) return ExpertArena{};
    ExpertArena a;
    a.buf = ArenaBuffer{r.base, frt_arena_total_bytes(&r), mode};
    a.blob_bytes = r.blob_bytes;
    a.stride = r.stride;
    a.n_layer = r.n_layer;
    a.n_expert = r.n_expert;
    return a;
}

inline void arena_free(ExpertArena& a) {
    if (a.buf.ptr) {
        frt_arena r = a.raw();
        frt_arena_free(&r);
    }
    a = ExpertArena{};
}

// Copies one planar host blob into (layer, expert) on `stream`.
inline void arena_upload(const ExpertArena& a, int layer, int expert, const void* host_blob, hipStream_t stream) {
    const frt_arena r = a.raw();
    detail::check(frt_arena_upload(&r, layer, expert, host_blob, stream), "arena_upload");
}

class CpuPool;   // the engine's (the HIP path needs no CPU pool; MoeFastHost keeps the pointer)

namespace q2_0 {
struct ExpertShape {
    int d_model, d_ff;
};
inline size_t mat_bytes(int rows, int cols) { return frt_q2_mat_bytes(rows, cols); }
inline size_t expert_bytes(ExpertShape s) { return frt_q2_expert_bytes(s.d_model, s.d_ff); }
// The planar repack of host memory; the reference returns a view, here the byte count written.
inline size_t repack(const void* ggml_rows, int rows, int cols, void* dst) {
    const size_t n = frt_q2_repack(ggml_rows, rows, cols, dst);
    if (n == 0) throw std::runtime_error(std::string("q2_0::repack: ") + frt_last_error());
    return n;
}
inline void repack_expert(const void* gate, const void* up, const void* down, ExpertShape s, void* blob) {
    detail::check(frt_q2_repack_expert(gate, up, down, s.d_model, s.d_ff, blob), "q2_0::repack_expert");
}
}  // namespace q2_0

namespace qwen4exp {

struct LoadStats {
    double seconds = 0;
    uint64_t bytes_read = 0;
};

// Reads the three expert slabs of every layer from the GGUF's shards (O_DIRECT), repacks each
// expert and uploads it into the HBM arena. Throws std::runtime_error on I/O errors or a missing
// tensor, as the reference does.
template <class GgufT, class SpecT>
LoadStats load_experts(const GgufT& g, const SpecT& s, ExpertArena& arena, int threads) {
    if (arena.blob_bytes != q2_0::expert_bytes({s.d_model, s.d_ff_expert}) || arena.n_layer != s.n_layer ||
        arena.n_expert != s.n_expert)
        throw std::runtime_error("load_experts: arena does not match the model");
    std::vector<frt_expert_slab> slabs(size_t(s.n_layer) * 3);
    static const char* const names[3] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    for (int l = 0; l < s.n_layer; ++l)
        for (int k = 0; k < 3; ++k) {
            const std::string n = "blk." + std::to_string(l) + "." + names[k] + ".weight";
            const auto* t = g.tensor(n);
            if (!t) throw std::runtime_error("missing " + n);
            slabs[size_t(l) * 3 + k] = frt_expert_slab{int(t->shard), uint64_t(t->file_offset)};
        }
    std::vector<const char*> paths;
    for (const auto& p : g.shards) paths.push_back(p.c_str());
    const frt_arena r = arena.raw();
    frt_load_stats st{};
    detail::check(frt_load_experts(paths.data(), int(paths.size()), slabs.data(), s.d_model, s.d_ff_expert, &r, threads, &st),
                  "load_experts");
    return LoadStats{st.seconds, st.bytes_read};
}

// The arena is device memory already: its device address.
inline const uint8_t* arena_register(const ExpertArena& arena) { return static_cast<const uint8_t*>(arena.buf.ptr); }

// A router or gate tensor in the GGUF type the model ships (ggml F32, F16, BF16, Q8_0) widened
// exactly to the fp32 layout the router takes (the reference reads it through ggml's linear(),
// arch/qwen4exp/blocks.hpp:85). Throws on an unsupported type.
inline void router_widen(hipStream_t stream, const void* src, int ggml_type, size_t count, float* dst) {
    detail::check(frt_router_widen(stream, src, ggml_type, count, dst), "router_widen");
}

inline void moe_route_topk(hipStream_t stream, const float* logits, int T, int E, int k, int32_t* ids, float* wts,
                           uint32_t* counts, uint32_t* tail_counts = nullptr, int tail_from = 1 << 30) {
    detail::check(frt_moe_route_topk(stream, logits, T, E, k, ids, wts, counts, tail_counts, tail_from),
                  "moe_route_topk");
}

// The reference sizes the scratch without d_model; this library also keeps the window's Q8
// activations there, so the size takes d_model (default: the largest supported, 16384).
inline size_t moe_hits_scratch_bytes(int K, int ff, int T = 1) {
    return frt_moe_hits_scratch_bytes(K, ff, T);
}

inline void moe_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const float* x, int n, int ff,
                     void* scratch, float* yh, hipStream_t stream, int T = 1) {
    detail::check(frt_moe_hits(hit_ptr, hit_n, K, x, n, ff, scratch, yh, stream, T), "moe_hits");
}

// The routing record of a layer call (blocks.hpp:280-283): top-k ids and their probabilities before
// renormalisation, [T][top_k].
struct MoeTrace {
    std::vector<int32_t> topk;
    std::vector<float> probs;
};

// One MoE layer on the HBM arena (router -> top-k -> routed experts + gated shared expert).
struct MoeLayer {
    frt_moe_layer desc{};

    MoeLayer() = default;
    MoeLayer(const uint8_t* experts, size_t stride, int n_expert, const uint8_t* shared, const float* router_w,
             const float* router_bias, const float* gate_w, int d_model, int d_ff, int top_k, bool norm_input = false) {
        desc = frt_moe_layer{experts, stride, n_expert, shared, router_w, router_bias, gate_w,
                             d_model, d_ff,   top_k,    norm_input ? FRT_LAYER_NORM_INPUT : 0, nullptr};
    }
    // the shared expert as the model's dense GGUF tensors (F32, F16, BF16 or Q8_0) instead of the
    // Q2_0 blob (frt_moe_layer.shared_dense)
    void set_shared_dense(int ggml_type, const void* gate, const void* up, const void* down, int shared_ff) {
        desc.shared_dense = 1;
        desc.shared_type = ggml_type;
        desc.shared_ff = shared_ff;
        desc.shared_gate = gate;
        desc.shared_up = up;
        desc.shared_down = down;
    }
    size_t workspace_bytes(int T) const { return frt_moe_layer_workspace_bytes(&desc, T); }
    // out [T][d_model] = (resid ? resid : 0) + moe(x); ids/wts [T][top_k], counts [E] optional;
    // tail_counts [E] += 1 per selection of tokens t >= tail_from (optional)
    void forward(const float* x, int T, float* out, void* ws, size_t ws_bytes, hipStream_t stream,
                 const float* resid = nullptr, int32_t* ids = nullptr, float* wts = nullptr, uint32_t* counts = nullptr,
                 uint32_t* tail_counts = nullptr, int tail_from = 1 << 30) const {
        detail::check(frt_moe_layer_forward_ex(&desc, x, T, resid, out, ids, wts, counts, tail_counts, tail_from, nullptr,
                                               ws, ws_bytes, stream),
                      "moe_layer_forward");
    }
    // forward() that also fills `trace` (synchronises the stream to read the record back).
    void forward_traced(const float* x, int T, float* out, void* ws, size_t ws_bytes, hipStream_t stream, MoeTrace& trace,
                        int32_t* ids, float* probs, const float* resid = nullptr) const {
        detail::check(frt_moe_layer_forward_ex(&desc, x, T, resid, out, ids, nullptr, nullptr, nullptr, 1 << 30, probs, ws,
                                               ws_bytes, stream),
                      "moe_layer_forward");
        const size_t nk = size_t(T) * desc.top_k;
        trace.topk.resize(nk);
        trace.probs.resize(nk);
        detail::hip_check(hipMemcpyAsync(trace.topk.data(), ids, nk * 4, hipMemcpyDeviceToHost, stream), "trace ids");
        detail::hip_check(hipMemcpyAsync(trace.probs.data(), probs, nk * 4, hipMemcpyDeviceToHost, stream), "trace probs");
        detail::hip_check(hipStreamSynchronize(stream), "trace");
    }
};

// ---- the expert cache: every expert resident; the cache is the arena (moe_fast.hpp:16-30)
struct ExpertCache {
    int n_slots = 0;
    size_t slot_bytes = 0;            // the arena stride
    uint8_t* slots = nullptr;         // the arena base (device)
    int32_t* table_dev = nullptr;     // [n_layer][n_expert] -> slot (the identity), device
    std::vector<int32_t> table;       // host mirror of table_dev
    std::vector<int32_t> owner;       // slot -> layer * n_expert + expert
};

// n_slots is what the engine could spare; every expert is resident whatever it asks for.
template <class SpecT>
ExpertCache alloc_expert_cache(const SpecT& s, int /*n_slots*/) {
    ExpertCache c;
    c.n_slots = s.n_layer * s.n_expert;
    c.table.resize(size_t(c.n_slots));
    c.owner.resize(size_t(c.n_slots));
    for (int i = 0; i < c.n_slots; ++i) c.table[size_t(i)] = c.owner[size_t(i)] = i;
    detail::hip_check(hipMalloc(reinterpret_cast<void**>(&c.table_dev), size_t(c.n_slots) * 4), "alloc_expert_cache");
    detail::hip_check(hipMemcpy(c.table_dev, c.table.data(), size_t(c.n_slots) * 4, hipMemcpyHostToDevice), "alloc_expert_cache");
    return c;
}
inline void free_expert_cache(ExpertCache& c) {
    if (c.table_dev) (void)hipFree(c.table_dev);
    c = ExpertCache{};
}
// Points the cache at the arena (slot i = arena blob i); nothing is uploaded.
template <class SpecT>
void expert_cache_fill(const SpecT& s, ExpertCache& cache, const ExpertArena& arena,
                       const std::vector<std::pair<int, int>>& /*order*/, hipStream_t /*stream*/) {
    if (arena.n_layer != s.n_layer || arena.n_expert != s.n_expert)
        throw std::runtime_error("expert_cache_fill: arena does not match the model");
    cache.slots = static_cast<uint8_t*>(arena.buf.ptr);
    cache.slot_bytes = arena.stride;
}

// Host-side state of moe_block_fast (moe_fast.hpp:32-77), with the layer descriptors and the
// workspace of the HIP path added (set_layer, once per layer at set-up).
struct MoeFastHost {
    const ExpertArena* arena = nullptr;
    CpuPool* pool = nullptr;
    bool doorbell = false;
    uint32_t seq = 0;
    bool db_failed = false;
    const uint8_t* arena_dev = nullptr;
    size_t arena_stride = 0;
    float pcie_frac = 0.0f;
    int pcie_max = 0;
    int max_window = 1;
    int window_T = 1;
    std::vector<int32_t> access;
    std::vector<int32_t> access_prev;
    int access_prev_T = 0;
    long hits = 0, misses = 0, gpu_misses = 0;
    double wait_s = 0, cpu_s = 0;
    // the HIP path
    std::vector<MoeLayer> layers;   // by layer index
    void* ws = nullptr;
    size_t ws_bytes = 0;

    void set_layer(int il, const MoeLayer& L) {
        if (il >= int(layers.size())) layers.resize(size_t(il) + 1);
        layers[size_t(il)] = L;
        const size_t need = L.workspace_bytes(max_window);
        if (need > ws_bytes) {
            if (ws) (void)hipFree(ws);
            ws = nullptr;
            ws_bytes = 0;
            detail::hip_check(hipMalloc(&ws, need), "MoeFastHost workspace");
            // zeroed: the address may have held a workspace the library has seen before
            detail::hip_check(hipMemset(ws, 0, need), "MoeFastHost workspace");
            ws_bytes = need;
        }
    }
};
template <class SpecT>
MoeFastHost alloc_moe_fast_host(const SpecT& /*s*/, int max_window = 1) {
    MoeFastHost h;
    h.max_window = max_window;
    return h;
}
inline void free_moe_fast_host(MoeFastHost& h) {
    if (h.ws) (void)hipFree(h.ws);
    h = MoeFastHost{};
}
// No misses: there is no miss server to start, and the pool stays free.
template <class SpecT>
void start_doorbell(const SpecT& /*s*/, MoeFastHost& h, int /*cpu*/) {
    h.doorbell = true;
}
inline void doorbell_begin_token(MoeFastHost& h, int T = 1) {
    h.window_T = T;
    ++h.seq;
}
template <class SpecT>
void doorbell_end_token(MoeFastHost& /*h*/, const SpecT& /*s*/) {}
inline bool doorbell_failed(const MoeFastHost& h) { return h.db_failed; }
inline void enable_pcie_misses(MoeFastHost& h, const ExpertArena& arena, float frac, int max_per_layer) {
    h.arena_dev = arena_register(arena);
    h.arena_stride = arena.stride;
    h.pcie_frac = frac;
    h.pcie_max = max_per_layer;
}

struct CachePolicyConfig {
    float decay = 0.7f;
    int decay_every = 4;
    float admit = 1.0f;
    float margin = 1.2f;
    int budget = 64;
    float seed_scale = 0.03f;
};
struct CacheManager {
    long steps = 0;
};
template <class SpecT>
CacheManager* create_cache_manager(const SpecT& /*s*/, ExpertCache& /*cache*/, const ExpertArena& /*arena*/,
                                   const CachePolicyConfig& /*cfg*/, const std::vector<uint32_t>& /*prior*/) {
    return new CacheManager{};
}
inline void destroy_cache_manager(CacheManager* m) { delete m; }
// Nothing to admit or evict: every expert is resident.
inline void cache_manager_step(CacheManager* m, const MoeFastHost& /*h*/, hipStream_t /*stream*/) {
    if (m) ++m->steps;
}
struct CacheStats {
    long swaps = 0, committed = 0;
};
inline CacheStats cache_manager_stats(const CacheManager* /*m*/) { return CacheStats{}; }
struct CacheCheck {
    long host_resident = 0, dev_resident = 0, table_mismatch = 0, owner_mismatch = 0, free_slots = 0, pending = 0;
};
inline CacheCheck cache_check(const ExpertCache& c, const CacheManager* /*m*/) {
    CacheCheck r;
    r.host_resident = r.dev_resident = c.n_slots;
    return r;
}

// T tokens: out [T][d_model] = routed experts + gated shared expert of layer il (registered with
// h.set_layer), every expert a hit. The stream is the context's.
template <class CtxT>
void moe_block_fast(const CtxT& c, int il, const float* x, const ExpertCache& /*cache*/, MoeFastHost& h, float* out,
                    int T = 1) {
    if (il < 0 || il >= int(h.layers.size())) throw std::runtime_error("moe_block_fast: layer not registered (set_layer)");
    h.layers[size_t(il)].forward(x, T, out, h.ws, h.ws_bytes, c.stream);
}

// ---- prefill chunks (moe_stream.hpp:18-36): the experts are resident, so nothing streams; the
// ExpertStream holds the layers' descriptors and one workspace for max_tokens.
struct ExpertStream {
    const ExpertArena* arena = nullptr;
    int max_tokens = 0;
    std::vector<MoeLayer> layers;
    void* ws = nullptr;
    size_t ws_bytes = 0;

    void set_layer(int il, const MoeLayer& L) {
        if (il >= int(layers.size())) layers.resize(size_t(il) + 1);
        layers[size_t(il)] = L;
        const size_t need = L.workspace_bytes(max_tokens);
        if (need > ws_bytes) {
            if (ws) (void)hipFree(ws);
            ws = nullptr;
            ws_bytes = 0;
            detail::hip_check(hipMalloc(&ws, need), "ExpertStream workspace");
            // zeroed: the address may have held a workspace the library has seen before
            detail::hip_check(hipMemset(ws, 0, need), "ExpertStream workspace");
            ws_bytes = need;
        }
    }
};
template <class SpecT>
ExpertStream* create_expert_stream(const SpecT& /*s*/, const ExpertArena& arena, int max_tokens) {
    auto* es = new ExpertStream{};
    es->arena = &arena;
    es->max_tokens = max_tokens;
    return es;
}
inline void destroy_expert_stream(ExpertStream* es) {
    if (!es) return;
    if (es->ws) (void)hipFree(es->ws);
    delete es;
}
inline size_t expert_stream_bytes(const ExpertStream* es) { return es ? es->ws_bytes : 0; }
// The workspace one layer of this model needs for max_tokens (the layers' own sizes add nothing more).
template <class SpecT>
size_t expert_stream_bytes_for(const SpecT& s, const ExpertArena& arena, int max_tokens) {
    frt_moe_layer d{};
    d.n_expert = s.n_expert;
    d.top_k = s.n_expert_used;
    d.d_model = s.d_model;
    d.d_ff = s.d_ff_expert;
    d.stride = arena.stride;
    return frt_moe_layer_workspace_bytes(&d, max_tokens);
}
inline void expert_stream_prefetch(ExpertStream* /*es*/, int /*il*/) {}   // resident: nothing to copy
template <class CtxT>
void moe_block_stream(const CtxT& c, int il, const float* x, int T, ExpertStream& es, float* out, uint32_t* counts,
                      uint32_t* tail_counts = nullptr, int tail_from = 1 << 30) {
    if (il < 0 || il >= int(es.layers.size())) throw std::runtime_error("moe_block_stream: layer not registered (set_layer)");
    if (T > es.max_tokens) throw std::runtime_error("moe_block_stream: T above max_tokens");
    es.layers[size_t(il)].forward(x, T, out, es.ws, es.ws_bytes, c.stream, nullptr, nullptr, nullptr, counts, tail_counts,
                                  tail_from);
}

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
