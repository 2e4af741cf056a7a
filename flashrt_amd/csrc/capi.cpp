// The C ABI (include/flashrt_moe.h): argument checks, workspace carving, error strings.
#include "common.hpp"

#include "../../include/flashrt_moe.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace frt {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

// ---- per-kernel timing
namespace {
struct Timing {
    bool on = false;
    std::vector<hipEvent_t> pool;
    size_t used = 0;   // events of the pool handed out since frt_timing_begin
    std::vector<std::pair<std::string, hipEvent_t>> marks;
    std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> kernels;   // start / stop at the kernel
    hipEvent_t take() {
        if (used == pool.size()) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) return nullptr;
            pool.push_back(e);
        }
        return pool[used++];
    }
};
Timing g_timing;
}  // namespace

bool timing_events(const char* kernel, hipEvent_t* start, hipEvent_t* stop) {
    Timing& t = g_timing;
    if (!t.on) return false;
    *start = t.take();
    *stop = t.take();
    if (!*start || !*stop) return false;
    t.kernels.push_back({kernel, {*start, *stop}});
    return true;
}

void timing_mark(hipStream_t stream, const char* kernel) {
    Timing& t = g_timing;
    if (!t.on) return;
    hipEvent_t e = t.take();
    if (!e || hipEventRecord(e, stream) != hipSuccess) return;
    t.marks.emplace_back(kernel, e);
}

// gen.hip
int router_widen(const void* src, int type, size_t count, float* dst, hipStream_t stream);
// route.hip
int router_logits(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                  float* logits, float* gate, hipStream_t stream, int norm, int8_t* xq, float* xd);
int rmsnorm(const float* x, int T, int n, float* u, hipStream_t stream);
int router_gemm(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                float* logits, float* gate, float* part, hipStream_t stream);
size_t router_gemm_ws_bytes(int T, int E, bool gate);
int quantize_q8(const float* x, int rows, int n, int8_t* xq, float* xd, _Float16* xhi, _Float16* xlo,
                hipStream_t stream);
int quantize_pairs(const float* x, int rows, int n, int np, int blk, _Float16* xhi, _Float16* xlo, hipStream_t stream);
int router_gemm_topk(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int n,
                     float* logits, float* gate, float* part, int K, int32_t* ids, float* wts, uint32_t* counts,
                     hipStream_t stream);
int route_topk(hipStream_t stream, const float* logits, int T, int E, int K, int32_t* ids, float* wts, uint32_t* counts,
               uint32_t* tail_counts, int tail_from);
bool router_fused_fits(int T, int n);
// decode.hip
size_t dec_scratch_bytes(int T, int K, int ff);
int dec_moe(const float* logits, const float* gate, int T, int E, int K, const uint8_t* arena, size_t stride,
            const uint8_t* shared_blob, const int8_t* xq, const float* xd, int n, int ff, int32_t* ids, float* wts,
            uint32_t* counts, const float* resid, float* out, void* scratch, hipStream_t stream,
            const float* prefetch = nullptr);
int dec_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const int8_t* xq, const float* xd, int n,
             int ff, void* scratch, float* yh, hipStream_t stream, int T);
int dec_check(int T, int K, int n, int ff);
size_t dec_window_bytes(int T, int K, int n, int ff);
int dec_window_fits(int T, int K, int ff);
bool decw_support(int T, int E, int K, int n, int ff);
int decw_layer(const float* x, int T, const float* W, const float* bias, const float* gate_w, int E, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared, int n, int ff, int norm, const float* resid,
               float* out, float* logits, float* gate, int32_t* ids, float* wts, uint32_t* counts, void* sync_ws,
               hipStream_t stream);
extern int g_decw_on;
int dec_window(const float* logits, int E, int32_t* ids, float* wts, uint32_t* counts, const float* gate, int T, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared_blob, const int8_t* xq, const float* xd, int n,
               int ff, const float* resid, float* out, void* scratch, hipStream_t stream);
// decode1.hip
size_t dec1_sync_bytes();
int dec1_eligible(int E, int K, int n, int ff);
int dec1_layer(const float* x, const float* W, const float* bias, const float* gate_w, int E, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared, int n, int ff, int norm, const float* resid,
               float* out, int32_t* ids, float* wts, uint32_t* counts, void* sync_ws, const float* next_w,
               hipStream_t stream);
int dec1_status(void* sync_ws, hipStream_t stream, uint32_t* err);
int dec1_support(int E, int K, int n, int ff);
const float* dec1_logits(const void* sync_ws, int* stride_floats);
// route.hip
int layer_trace(const float* lg, int ls, const int32_t* ids, int T, int E, int K, uint32_t* tail_counts, int tail_from,
                float* probs, hipStream_t stream);
int dec1_stack(const frt_moe_layer* L, int n_layer, const float* x, float* out, int32_t* ids, float* wts,
               void* sync_ws, hipStream_t stream);
int dec1_take_timeout();
// decode2.hip
int dec2_support(int E, int K, int n, int ff, int n_layer);
int dec2_layer(const float* x, const float* W, const float* bias, const float* gate_w, int E, int K,
               const uint8_t* arena, size_t stride, const uint8_t* shared, int n, int ff, int norm, const float* resid,
               float* out, int32_t* ids, float* wts, uint32_t* counts, void* sync_ws, const float* next_w,
               hipStream_t stream);
int dec2_stack(const frt_moe_layer* L, int n_layer, const float* x, float* out, int32_t* ids, float* wts,
               void* sync_ws, hipStream_t stream);
extern int g_dec2_on;
extern uint64_t* g_dec2_stamps;
extern int g_route8;
extern thread_local bool g_dec1_no_alloc;
extern int g_dec1_on;
extern uint64_t g_dec1_ticks;
extern int g_dec1_grid_cap;
// prefill.hip
size_t pf_workspace_bytes(int T, int K, int n, int ff, int E, bool shared, bool own_yd);
int pf_run(const uint8_t* experts, size_t stride, int E, int n, int ff, const float* x, const int32_t* ids, int T, int K,
           void* yd, void* ws, size_t ws_bytes, hipStream_t stream, int block64, int yd_bf16);
int pf_moe(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, int n, int ff, const float* x,
           const int32_t* ids, const float* wts, const float* gate, int T, int K, const float* resid, float* out,
           void* ws, size_t ws_bytes, hipStream_t stream);
int pf_dispatch(const int32_t* ids, int T, int K, int E, int32_t* bounds, int32_t* tok_of, int32_t* slot_of, void* ws,
                size_t ws_bytes, hipStream_t stream);
size_t pf_dispatch_ws_bytes(int T, int K, int E);
int pf_check(int T, int K, int n, int ff, int E);
// gen.hip
int gen_experts(uint64_t seed, int cfg, int layer, int e0, int count, int tensor_base, int n, int ff, float sd,
                uint8_t* dst, size_t stride, hipStream_t stream);
int gen_normal(uint64_t seed, int cfg, int layer, int tensor, float sd, float* dst, size_t count, int round_bf16,
               hipStream_t stream);
int gen_correlated(uint64_t seed, int cfg, int layer, int tensor0, int T, int n, float rho, float* dst,
                   hipStream_t stream);
void gen_zipf_bias(uint64_t seed, int cfg, int layer, int E, float s, float alpha, float* bias);

// shexp.hip
bool shexp_type_ok(int type);
bool shexp_shape_ok(int n, int ffs);
size_t shexp_ws_bytes(int T, int n, int ffs);
int shexp_run(int type, const void* g, const void* u, const void* d, int n, int ffs, const float* x, const int8_t* xq,
              const float* xd, int T, float* sh, void* ws, hipStream_t stream);
int hits_from_ids(const int32_t* ids, int T, int K, const uint8_t* arena, size_t stride, const uint8_t* shared,
                  const uint8_t** hit_ptr, int32_t* hit_n, hipStream_t stream);
int slot_combine(int T, int K, int S, int n, const int32_t* ids, const float* wts, const float* Y, const float* sh,
                 size_t sh_stride, const float* gate, const float* resid, float* out, hipStream_t stream);
// decode.hip
bool dec_shape_templated(int n, int ff);
bool dec_shape_generic(int n, int ff);

constexpr int kDecodeMaxT = 4;

// moe_hits runs a window in launches of at most hits_chunk(T, K, ff) tokens: 8 (the reference's
// kMaxWindow) as long as the launch has at most 128 (token, slot) items (K <= 16 for 8 tokens); each
// launch reads each of its distinct blobs once per four of its tokens
static int hits_chunk(int T, int K, int ff) {
    (void)ff;
    int c = 8;
    const int k = K > 0 ? K : 1;
    while (c > 1 && c * k > 128) --c;
    return T < c ? T : c;
}
// decode-side scratch for moe_hits: x quantized (T rows of up to kHitsMaxN values) ahead of the dec
// scratch of one chunk; the size does not depend on the call's n (as the reference's, moe_fast.hpp:134)
constexpr int kHitsMaxN = 16384;
static size_t hits_bytes(int K, int ff, int T, int n) {
    return up256(size_t(T) * n) + up256(size_t(T) * (n / kQ8) * 4) + dec_scratch_bytes(hits_chunk(T, K, ff), K, ff);
}

struct LayerWs {
    void* sync;    // the single-token layer's sync region (always first, so no other path overwrites it)
    float* logits;
    float* gate;
    float* u;      // normalised input (prefill with FRT_LAYER_NORM_INPUT)
    float* part;   // router GEMM split partial sums (prefill)
    int32_t* ids;
    float* wts;
    int8_t* xq;
    float* xd;
    void* rest;
    size_t rest_bytes;
    size_t bytes;
};

// A verify window of 5 .. 8 tokens (the reference's kMaxWindow) goes through the decode GEMV kernels
// (router + fused Q8_0, top-k, one moe_hits launch, combine) when it fits one hits launch and the
// router's fused quantization; larger windows take the prefill path.
extern int g_router_mfma;
int g_window_min_t = 2;   // windows of at least this many tokens take the window path (measured faster from 2)
static bool window_path(const frt_moe_layer& L, int T) {
    const int K = L.top_k, n = L.d_model;
    if (T < g_window_min_t && T <= kDecodeMaxT && T * K <= 63) return false;   // the grouped decode path
    return T <= 8 && dec_window_fits(T, K, L.d_ff) && router_fused_fits(T, n) && dec_check(1, K, n, L.d_ff) == kOk;
}

// ---- the slot path of a layer: the routed experts as per-slot outputs (moe_hits for windows of up to 8
// tokens, moe_q2::run beyond), the shared expert, then the slot combine. Taken by a layer whose shared
// expert is given as dense GGUF tensors (frt_moe_layer.shared_dense; shexp.hip), and by windows whose
// shape is outside the templated decode kernels (n a multiple of 512, ff a multiple of 64 up to 4096:
// the reference's moe_hits envelope), where the Q2_0 shared expert is moe_hits slot K.
struct DenseWs {
    float* u;                  // the layer input (normalised with FRT_LAYER_NORM_INPUT)
    int8_t* xq;
    float* xd;
    float* part;               // router GEMM partials (prefill)
    const uint8_t** hit_ptr;   // [T][K] (windows)
    int32_t* hit_n;            // [T]
    float* Y;                  // per-slot outputs [T][K][n]
    float* sh;                 // shared expert output [T][n]
    void* shws;
    void* rws;                 // moe_hits scratch or moe_q2 workspace
    size_t rws_bytes;
    size_t end;                // bytes from the layer workspace's start
};
static bool dense_small(const frt_moe_layer& L, int T) {
    const int S = L.shared_dense ? L.top_k : L.top_k + 1;   // moe_hits slots per token
    return T <= 8 && S <= 32 && (dec_shape_templated(L.d_model, L.d_ff) || dec_shape_generic(L.d_model, L.d_ff));
}
// the slot path: a dense shared expert, or a window of a shape the templated decode kernels lack
static bool slot_path(const frt_moe_layer& L, int T) {
    if (L.shared_dense) return true;
    return T <= 8 && !dec_shape_templated(L.d_model, L.d_ff) && dense_small(L, T) &&
           router_fused_fits(T, L.d_model);
}
static DenseWs dense_carve(uint8_t* p0, uint8_t* p, const frt_moe_layer& L, int T) {
    DenseWs w{};
    auto take = [&](size_t b) {
        uint8_t* r = p;
        p += up256(b);
        return r;
    };
    const int E = L.n_expert, K = L.top_k, n = L.d_model, ff = L.d_ff;
    w.u = reinterpret_cast<float*>(take(size_t(T) * n * 4));
    w.xq = reinterpret_cast<int8_t*>(take(size_t(T) * n));
    w.xd = reinterpret_cast<float*>(take(size_t(T) * (n / kQ8) * 4));
    w.hit_ptr = reinterpret_cast<const uint8_t**>(take(size_t(T) * (K + 1) * 8));
    w.hit_n = reinterpret_cast<int32_t*>(take(size_t(T) * 4));
    w.Y = reinterpret_cast<float*>(take(size_t(T) * (K + 1) * n * 4));
    w.sh = reinterpret_cast<float*>(take(size_t(T) * n * 4));
    w.shws = take(shexp_ws_bytes(T, n, L.shared_ff > 0 ? L.shared_ff : 64));
    if (dense_small(L, T)) {
        const int S = L.shared_dense ? K : K + 1;
        w.rws_bytes = dec_scratch_bytes(hits_chunk(T, S, ff), S, ff);
    } else {
        w.part = reinterpret_cast<float*>(take(router_gemm_ws_bytes(T, E, true)));
        w.rws_bytes = pf_workspace_bytes(T, K, n, ff, E, false, false);
    }
    w.rws = take(w.rws_bytes);
    w.end = size_t(p - p0);
    return w;
}

static int dense_layer(const frt_moe_layer& L, const LayerWs& lw, const DenseWs& w, const float* x, int T,
                       const float* resid, float* out, int32_t* ids, float* wts, uint32_t* counts, hipStream_t s) {
    const int E = L.n_expert, K = L.top_k, n = L.d_model, ff = L.d_ff, ffs = L.shared_ff;
    const bool dense = L.shared_dense != 0;
    if (dense) {
        if (!L.shared_gate || !L.shared_up || !L.shared_down) return set_error(kErrNull, "moe_layer: shared tensors missing");
        if (!shexp_type_ok(L.shared_type))
            return set_error(kErrShape, "moe_layer: shared expert type %d (F32, F16, BF16 or Q8_0)", L.shared_type);
        if (!shexp_shape_ok(n, ffs)) return set_error(kErrShape, "moe_layer: shared_ff=%d n=%d", ffs, n);
    }
    const bool small = dense_small(L, T);
    const int S = dense ? K : K + 1;   // moe_hits slots per token (the Q2_0 shared expert as slot K)
    if (!dense && !small) return set_error(kErrShape, "moe_layer: slot path for T=%d K=%d n=%d ff=%d", T, K, n, ff);
    if (!small)
        if (int rc = pf_check(T, K, n, ff, E)) return rc;
    const float* u = x;
    if (L.flags & FRT_LAYER_NORM_INPUT) {
        if (int rc = rmsnorm(x, T, n, w.u, s)) return rc;
        u = w.u;
        timing_mark(s, "rmsnorm");
    }
    if (small && router_fused_fits(T, n)) {
        if (int rc = router_logits(u, T, L.router_w, L.router_bias, L.gate_w, E, n, lw.logits, lw.gate, s, 0, w.xq, w.xd))
            return rc;
    } else {
        if (small) {
            if (int rc = router_logits(u, T, L.router_w, L.router_bias, L.gate_w, E, n, lw.logits, lw.gate, s, 0, nullptr,
                                       nullptr))
                return rc;
        } else if (int rc = router_gemm_topk(u, T, L.router_w, L.router_bias, L.gate_w, E, n, lw.logits, lw.gate,
                                             w.part, K, ids, wts, counts, s)) {
            return rc;
        }
        if (small || (dense && L.shared_type == FRT_GGML_Q8_0))
            if (int rc = quantize_q8(u, T, n, w.xq, w.xd, nullptr, nullptr, s)) return rc;
    }
    timing_mark(s, "router");
    if (small)   // (the GEMM path selected already)
        if (int rc = route_topk(s, lw.logits, T, E, K, ids, wts, counts, nullptr, 1 << 30)) return rc;
    timing_mark(s, "route_topk");
    if (small) {
        if (int rc = hits_from_ids(ids, T, K, L.experts, L.stride, dense ? nullptr : L.shared, w.hit_ptr, w.hit_n, s))
            return rc;
        const int tc = hits_chunk(T, S, ff);
        for (int t0 = 0; t0 < T; t0 += tc) {
            const int tn = T - t0 < tc ? T - t0 : tc;
            if (int rc = dec_hits(w.hit_ptr + size_t(t0) * S, w.hit_n + t0, S, w.xq + size_t(t0) * n,
                                  w.xd + size_t(t0) * (n / kQ8), n, ff, w.rws, w.Y + size_t(t0) * S * n, s, tn))
                return rc;
        }
    } else if (int rc = pf_run(L.experts, L.stride, E, n, ff, u, ids, T, K, w.Y, w.rws, w.rws_bytes, s, 0, 0)) {
        return rc;
    }
    const float* sh = w.Y + size_t(K) * n;   // the Q2_0 shared expert: slot K of each token
    size_t sh_stride = size_t(S) * n;
    if (dense) {
        if (int rc = shexp_run(L.shared_type, L.shared_gate, L.shared_up, L.shared_down, n, ffs, u, w.xq, w.xd, T, w.sh,
                               w.shws, s))
            return rc;
        timing_mark(s, "shared_expert");
        sh = w.sh;
        sh_stride = size_t(n);
    }
    if (int rc = slot_combine(T, K, S, n, ids, wts, w.Y, sh, sh_stride, lw.gate, resid, out, s)) return rc;
    timing_mark(s, "combine");
    return kOk;
}

static LayerWs layer_carve(void* base, const frt_moe_layer& L, int T, size_t total) {
    LayerWs w{};
    uint8_t* p = static_cast<uint8_t*>(base);
    auto take = [&](size_t b) {
        uint8_t* r = p;
        p += up256(b);
        return r;
    };
    const int E = L.n_expert, K = L.top_k, n = L.d_model, ff = L.d_ff;
    w.sync = take(dec1_sync_bytes());
    w.logits = reinterpret_cast<float*>(take(size_t(T) * E * 4));
    w.gate = reinterpret_cast<float*>(take(size_t(T) * 4));
    w.ids = reinterpret_cast<int32_t*>(take(size_t(T) * K * 4));
    w.wts = reinterpret_cast<float*>(take(size_t(T) * K * 4));
    // the decode window paths a call of T tokens can take, whatever "window_min_t" is set to: the
    // workspace holds the larger of their layouts, so a size queried once stays valid after the option
    // changes (both carve xq and xd first, then their own scratch)
    if (slot_path(L, T)) {   // the slot path (dense_layer)
        const DenseWs d = dense_carve(static_cast<uint8_t*>(base), p, L, T);
        w.bytes = d.end;
        return w;
    }
    const bool dec_ok = T <= kDecodeMaxT && T * K <= 63;
    const bool win_ok = T <= 8 && dec_window_fits(T, K, ff) && router_fused_fits(T, n) && dec_check(1, K, n, ff) == kOk;
    if (dec_ok || win_ok) {
        w.xq = reinterpret_cast<int8_t*>(take(size_t(T) * n));
        w.xd = reinterpret_cast<float*>(take(size_t(T) * (n / kQ8) * 4));
        const size_t db = dec_ok ? dec_scratch_bytes(T, K, ff) : 0, wb = win_ok ? dec_window_bytes(T, K, n, ff) : 0;
        w.rest_bytes = db > wb ? db : wb;
    } else {
        if (L.flags & FRT_LAYER_NORM_INPUT) w.u = reinterpret_cast<float*>(take(size_t(T) * n * 4));
        w.part = reinterpret_cast<float*>(take(router_gemm_ws_bytes(T, E, true)));
        w.rest_bytes = pf_workspace_bytes(T, K, n, ff, E, true, true);
    }
    w.rest = take(w.rest_bytes);
    w.bytes = size_t(p - static_cast<uint8_t*>(base));
    (void)total;
    return w;
}

// ---- the allocation-free decode entry point's workspace: a file-scope device array, one copy per
// GPU, held until the process ends. Host code never passes the array's name to a kernel or a copy:
// it uses the device address hipGetSymbolAddress returns, looked up once per device.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

static int scratch_ptr(void** out) {
    int dev = 0;
    FRT_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return set_error(kErrShape, "noalloc scratch: device %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {   // once per device, with that device current
        void* p = nullptr;
        FRT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return set_error(kErrHip, "noalloc scratch: no device address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}

}  // namespace frt

using namespace frt;

extern "C" {

const char* frt_last_error(void) { return g_err; }

void frt_timing_begin(void) {
    g_timing.on = true;
    g_timing.marks.clear();
    g_timing.kernels.clear();
    g_timing.used = 0;
}

// Durations between consecutive marks of one stream's launches, summed per kernel name (a mark
// named "begin" opens each call); kernels launched with their own start / stop events report those
// instead. Writes up to max entries; returns the number of kernel names.
int frt_timing_end(char* names, int name_len, double* total_ms, int* launches, int max) {
    Timing& t = g_timing;
    t.on = false;
    if (!t.marks.empty()) FRT_HIP(hipEventSynchronize(t.marks.back().second));
    std::map<std::string, std::pair<double, int>> acc;
    std::vector<std::string> order;
    for (size_t i = 1; i < t.marks.size(); ++i) {
        const std::string& k = t.marks[i].first;
        if (k == "begin") continue;
        float ms = 0.0f;
        FRT_HIP(hipEventElapsedTime(&ms, t.marks[i - 1].second, t.marks[i].second));
        if (!acc.count(k)) order.push_back(k);
        acc[k].first += ms;
        acc[k].second += 1;
    }
    // kernels with events of their own: their start-to-stop times replace the intervals
    std::map<std::string, std::pair<double, int>> own;
    for (const auto& ke : t.kernels) {
        FRT_HIP(hipEventSynchronize(ke.second.second));
        float ms = 0.0f;
        FRT_HIP(hipEventElapsedTime(&ms, ke.second.first, ke.second.second));
        own[ke.first].first += ms;
        own[ke.first].second += 1;
        if (!acc.count(ke.first)) order.push_back(ke.first);
    }
    for (const auto& o : own) acc[o.first] = o.second;
    int n = 0;
    for (const auto& k : order) {
        if (n >= max) break;
        std::snprintf(names + size_t(n) * name_len, size_t(name_len), "%s", k.c_str());
        total_ms[n] = acc[k].first;
        launches[n] = acc[k].second;
        ++n;
    }
    t.marks.clear();
    t.kernels.clear();
    t.used = 0;
    return n;
}
const char* frt_version(void) { return "flashrt-mi355x 0.1 (gfx950)"; }

size_t frt_q2_mat_bytes(int rows, int cols) { return mat_bytes(rows, cols); }
size_t frt_q2_expert_bytes(int d_model, int d_ff) { return expert_bytes(d_model, d_ff); }

int frt_arena_alloc(int n_layer, int n_expert, size_t blob_bytes, frt_arena* out) {
    if (!out) return set_error(kErrNull, "arena_alloc: null out");
    *out = frt_arena{};
    if (n_layer < 1 || n_expert < 1 || blob_bytes == 0) return set_error(kErrShape, "arena_alloc: bad shape");
    const size_t stride = (blob_bytes + 4095) & ~size_t(4095);
    void* p = nullptr;
    FRT_HIP(hipMalloc(&p, stride * size_t(n_layer) * size_t(n_expert)));
    *out = frt_arena{static_cast<uint8_t*>(p), blob_bytes, stride, n_layer, n_expert};
    return kOk;
}

int frt_arena_free(frt_arena* a) {
    if (!a) return set_error(kErrNull, "arena_free: null");
    if (a->base) FRT_HIP(hipFree(a->base));
    *a = frt_arena{};
    return kOk;
}

uint8_t* frt_arena_blob(const frt_arena* a, int layer, int expert) {
    return a->base + (size_t(layer) * a->n_expert + expert) * a->stride;
}
size_t frt_arena_total_bytes(const frt_arena* a) { return size_t(a->n_layer) * a->n_expert * a->stride; }

int frt_arena_upload(const frt_arena* a, int layer, int expert, const void* host_blob, void* stream) {
    if (!a || !a->base || !host_blob) return set_error(kErrNull, "arena_upload: null");
    if (layer < 0 || layer >= a->n_layer || expert < 0 || expert >= a->n_expert) return set_error(kErrShape, "arena_upload: index");
    FRT_HIP(hipMemcpyAsync(frt_arena_blob(a, layer, expert), host_blob, a->blob_bytes, hipMemcpyHostToDevice,
                           static_cast<hipStream_t>(stream)));
    return kOk;
}

int frt_moe_route_topk(void* stream, const float* logits, int T, int E, int k, int32_t* ids, float* wts,
                       uint32_t* counts, uint32_t* tail_counts, int tail_from) {
    return route_topk(static_cast<hipStream_t>(stream), logits, T, E, k, ids, wts, counts, tail_counts, tail_from);
}

int frt_router_logits(void* stream, const float* x, int T, const float* W, const float* bias, const float* gate_w,
                      int E, int n, float* logits, float* gate) {
    return router_logits(x, T, W, bias, gate_w, E, n, logits, gate, static_cast<hipStream_t>(stream), 0, nullptr, nullptr);
}

size_t frt_router_gemm_workspace_bytes(int T, int E, int has_gate) {
    return T < 1 || E < 1 ? 0 : router_gemm_ws_bytes(T, E, has_gate != 0);
}

int frt_router_logits_gemm(void* stream, const float* x, int T, const float* W, const float* bias, const float* gate_w,
                           int E, int n, float* logits, float* gate, void* ws, size_t ws_bytes) {
    if (!x || !W || !logits || !ws) return set_error(kErrNull, "router_logits_gemm: null pointer");
    if (T < 1 || E < 1 || E > 4096) return set_error(kErrShape, "router_logits_gemm: T=%d E=%d", T, E);
    if (ws_bytes < router_gemm_ws_bytes(T, E, gate_w != nullptr))
        return set_error(kErrWorkspace, "router_logits_gemm: workspace %zu < %zu", ws_bytes,
                         router_gemm_ws_bytes(T, E, gate_w != nullptr));
    return router_gemm(x, T, W, bias, gate_w, E, n, logits, gate, static_cast<float*>(ws), static_cast<hipStream_t>(stream));
}

int frt_router_widen(void* stream, const void* src, int type, size_t count, float* dst) {
    return router_widen(src, type, count, dst, static_cast<hipStream_t>(stream));
}

int frt_quantize_q8(void* stream, const float* x, int rows, int n, int8_t* xq, float* xd) {
    if (!x || !xq || !xd) return set_error(kErrNull, "quantize_q8: null pointer");
    return quantize_q8(x, rows, n, xq, xd, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

int frt_quantize_pairs(void* stream, const float* x, int rows, int n, int block, uint16_t* xhi, uint16_t* xlo) {
    if (!x || !xhi || !xlo) return set_error(kErrNull, "quantize_pairs: null pointer");
    return quantize_pairs(x, rows, n, (n + 511) & ~511, block, reinterpret_cast<_Float16*>(xhi),
                          reinterpret_cast<_Float16*>(xlo), static_cast<hipStream_t>(stream));
}

size_t frt_moe_dispatch_workspace_bytes(int T, int K, int E) { return pf_dispatch_ws_bytes(T, K, E); }
int frt_moe_dispatch(void* stream, const int32_t* ids, int T, int K, int E, int32_t* bounds, int32_t* tok_of,
                     int32_t* slot_of, void* ws, size_t ws_bytes) {
    if (!ids || !bounds || !tok_of || !slot_of || !ws) return set_error(kErrNull, "dispatch: null pointer");
    return pf_dispatch(ids, T, K, E, bounds, tok_of, slot_of, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

size_t frt_moe_q2_workspace_bytes(int T, int K, int n, int ff, int E) {
    return pf_workspace_bytes(T, K, n, ff, E, false, false);
}
int frt_moe_q2_run(const uint8_t* experts, size_t stride, int E, int n, int ff, const float* x, const int32_t* ids,
                   int T, int K, void* yd, void* ws, size_t ws_bytes, void* stream, int block64, int yd_bf16) {
    return pf_run(experts, stride, E, n, ff, x, ids, T, K, yd, ws, ws_bytes, static_cast<hipStream_t>(stream), block64,
                  yd_bf16);
}

size_t frt_moe_hits_scratch_bytes(int K, int ff, int T) { return hits_bytes(K, ff, T, kHitsMaxN); }
int frt_moe_hits(const uint8_t* const* hit_ptr, const int32_t* hit_n, int K, const float* x, int n, int ff,
                 void* scratch, float* yh, void* stream, int T) {
    if (!hit_ptr || !hit_n || !x || !scratch || !yh) return set_error(kErrNull, "moe_hits: null pointer");
    if (T < 1 || K < 1 || K > 32) return set_error(kErrShape, "moe_hits: T=%d K=%d", T, K);
    const int tc = hits_chunk(T, K, ff);
    if (n > kHitsMaxN || (!dec_shape_templated(n, ff) && !dec_shape_generic(n, ff)))   // (moe_fast.cu:557)
        return set_error(kErrShape, "moe_hits: n=%d ff=%d (n %% 512 == 0, ff %% 64 == 0, ff <= 4096)", n, ff);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t* p = static_cast<uint8_t*>(scratch);
    int8_t* xq = reinterpret_cast<int8_t*>(p);
    p += up256(size_t(T) * n);
    float* xd = reinterpret_cast<float*>(p);
    p += up256(size_t(T) * (n / kQ8) * 4);
    if (int rc = quantize_q8(x, T, n, xq, xd, nullptr, nullptr, s)) return rc;
    for (int t0 = 0; t0 < T; t0 += tc) {   // chunks in stream order share the dec scratch
        const int tn = T - t0 < tc ? T - t0 : tc;
        if (int rc = dec_hits(hit_ptr + size_t(t0) * K, hit_n + t0, K, xq + size_t(t0) * n, xd + size_t(t0) * (n / kQ8),
                              n, ff, p, yh + size_t(t0) * K * n, s, tn))
            return rc;
    }
    return kOk;
}

size_t frt_moe_layer_workspace_bytes(const frt_moe_layer* L, int T) {
    if (!L || T < 1) return 0;
    return layer_carve(nullptr, *L, T, 0).bytes + 256;
}

int frt_moe_layer_forward(const frt_moe_layer* L, const float* x, int T, const float* resid, float* out, int32_t* ids,
                          float* wts, uint32_t* counts, void* ws, size_t ws_bytes, void* stream) {
    if (!L || !x || !out || !ws) return set_error(kErrNull, "moe_layer: null pointer");
    if (!L->experts || (!L->shared && !L->shared_dense) || !L->router_w || !L->gate_w)
        return set_error(kErrNull, "moe_layer: layer weights missing");
    if (T < 1) return set_error(kErrShape, "moe_layer: T=%d", T);
    if (int rc = dec1_take_timeout()) return rc;
    const int E = L->n_expert, K = L->top_k, n = L->d_model, ff = L->d_ff;
    if (E < 1 || E > 1024 || K < 1 || K > 32 || K > E) return set_error(kErrShape, "moe_layer: E=%d K=%d", E, K);
    if (L->stride < expert_bytes(n, ff)) return set_error(kErrShape, "moe_layer: stride %zu < blob %zu", L->stride, expert_bytes(n, ff));
    const LayerWs w = layer_carve(ws, *L, T, ws_bytes);
    if (w.bytes > ws_bytes) return set_error(kErrWorkspace, "moe_layer: workspace %zu < %zu", ws_bytes, w.bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    int32_t* ids_o = ids ? ids : w.ids;
    float* wts_o = wts ? wts : w.wts;
    const int norm = (L->flags & FRT_LAYER_NORM_INPUT) ? 1 : 0;
    timing_mark(s, "begin");
    if (slot_path(*L, T)) {
        uint8_t* b = static_cast<uint8_t*>(ws);
        uint8_t* p = b + (reinterpret_cast<uint8_t*>(w.wts) - b) + up256(size_t(T) * K * 4);
        const DenseWs d = dense_carve(b, p, *L, T);
        return dense_layer(*L, w, d, x, T, resid, out, ids_o, wts_o, counts, s);
    }
    if (T == 1 && g_dec1_on && dec2_support(E, K, n, ff, 1))   // one persistent launch, joins split by XCD
        return dec2_layer(x, L->router_w, L->router_bias, L->gate_w, E, K, L->experts, L->stride, L->shared, n, ff,
                          norm, resid, out, ids_o, wts_o, counts, w.sync, L->next_router_w, s);
    if (T == 1 && g_dec1_on && dec1_support(E, K, n, ff) >= 1)   // the whole layer in one persistent launch
        return dec1_layer(x, L->router_w, L->router_bias, L->gate_w, E, K, L->experts, L->stride, L->shared, n, ff,
                          norm, resid, out, ids_o, wts_o, counts, w.sync, L->next_router_w, s);
    if (T >= 2 && T >= g_window_min_t && decw_support(T, E, K, n, ff))   // a window of 2-4 tokens in one persistent launch
        return decw_layer(x, T, L->router_w, L->router_bias, L->gate_w, E, K, L->experts, L->stride, L->shared, n, ff,
                          norm, resid, out, w.logits, w.gate, ids_o, wts_o, counts, w.sync, s);
    if (!window_path(*L, T) && T <= kDecodeMaxT && T * K <= 63) {
        if (int rc = dec_check(T, K, n, ff)) return rc;
        // router logits, the shared gate, the RMS scale and Q8_0 of the input in one launch
        if (int rc = router_logits(x, T, L->router_w, L->router_bias, L->gate_w, E, n, w.logits, w.gate, s, norm, w.xq,
                                   w.xd))
            return rc;
        timing_mark(s, "router_quant");
        return dec_moe(w.logits, w.gate, T, E, K, L->experts, L->stride, L->shared, w.xq, w.xd, n, ff, ids_o, wts_o,
                       counts, resid, out, w.rest, s, L->next_router_w);
    }
    if (window_path(*L, T)) {
        if (int rc = router_logits(x, T, L->router_w, L->router_bias, L->gate_w, E, n, w.logits, w.gate, s, norm, w.xq,
                                   w.xd))
            return rc;
        timing_mark(s, "router_quant");
        return dec_window(w.logits, E, ids_o, wts_o, counts, w.gate, T, K, L->experts, L->stride, L->shared, w.xq, w.xd,
                          n, ff, resid, out, w.rest, s);
    }
    if (int rc = pf_check(T, K, n, ff, E)) return rc;
    const float* xin = x;
    if (norm) {
        if (int rc = rmsnorm(x, T, n, w.u, s)) return rc;
        xin = w.u;
        timing_mark(s, "rmsnorm");
    }
    // router logits and the shared expert's gate logit (row E) as one K-split GEMM, then the top-k
    // (with the split's combine where E <= 512)
    if (int rc = router_gemm_topk(xin, T, L->router_w, L->router_bias, L->gate_w, E, n, w.logits, w.gate, w.part, K,
                                  ids_o, wts_o, counts, s))
        return rc;
    timing_mark(s, "route_topk");
    return pf_moe(L->experts, L->stride, E, L->shared, n, ff, xin, ids_o, wts_o, w.gate, T, K, resid, out, w.rest,
                  w.rest_bytes, s);
}

size_t frt_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int frt_moe_layer_forward_noalloc(const frt_moe_layer* L, const float* x, int T, const float* resid, float* out,
                                  int32_t* ids, float* wts, uint32_t* counts, void* stream) {
    if (!L) return set_error(kErrNull, "moe_layer_forward_noalloc: null layer");
    if (T < 1 || T > kDecodeMaxT || T * L->top_k > 63)
        return set_error(kErrShape, "moe_layer_forward_noalloc: decode windows only (1 <= T <= %d, T * K <= 63), "
                                    "got T=%d K=%d", kDecodeMaxT, T, L->top_k);
    const size_t need = frt_moe_layer_workspace_bytes(L, T);
    if (need == 0 || need > kNoAllocScratchBytes)
        return set_error(kErrWorkspace, "moe_layer_forward_noalloc: needs %zu bytes of workspace; the static "
                                        "scratch holds %zu", need, kNoAllocScratchBytes);
    void* p = nullptr;
    if (int rc = scratch_ptr(&p)) return rc;
    struct NoAllocScope {   // the persistent path then allocates nothing (no host time-out flag)
        NoAllocScope() { g_dec1_no_alloc = true; }
        ~NoAllocScope() { g_dec1_no_alloc = false; }
    } scope;
    return frt_moe_layer_forward(L, x, T, resid, out, ids, wts, counts, p, kNoAllocScratchBytes, stream);
}

int frt_noalloc_sync_error(void* stream) {
    void* p = nullptr;
    if (int rc = scratch_ptr(&p)) return rc;
    uint32_t err = 0;
    if (int rc = dec1_status(p, static_cast<hipStream_t>(stream), &err)) return rc;
    return err ? 1 : 0;
}

size_t frt_moe_stack_workspace_bytes(const frt_moe_layer* layers, int n_layer) {
    if (!layers || n_layer < 1) return 0;
    return frt_moe_layer_workspace_bytes(&layers[0], 1) + 2 * up256(size_t(layers[0].d_model) * 4);
}

int frt_moe_stack_forward(const frt_moe_layer* layers, int n_layer, const float* x, float* out, int32_t* ids,
                          float* wts, void* ws, size_t ws_bytes, void* stream) {
    if (!layers || !x || !out || !ws) return set_error(kErrNull, "moe_stack: null pointer");
    if (n_layer < 1) return set_error(kErrShape, "moe_stack: n_layer=%d", n_layer);
    if (int rc = dec1_take_timeout()) return rc;
    const frt_moe_layer& L0 = layers[0];
    for (int l = 0; l < n_layer; ++l) {
        const frt_moe_layer& Ll = layers[l];
        if (!Ll.experts || (!Ll.shared && !Ll.shared_dense) || !Ll.router_w || !Ll.gate_w)
            return set_error(kErrNull, "moe_stack: layer %d weights missing", l);
        if (Ll.n_expert != L0.n_expert || Ll.top_k != L0.top_k || Ll.d_model != L0.d_model || Ll.d_ff != L0.d_ff ||
            Ll.stride != L0.stride || Ll.flags != L0.flags)
            return set_error(kErrShape, "moe_stack: layer %d differs in shape, stride or flags from layer 0", l);
    }
    const size_t need = frt_moe_stack_workspace_bytes(layers, n_layer);
    if (ws_bytes < need) return set_error(kErrWorkspace, "moe_stack: workspace %zu < %zu", ws_bytes, need);
    const int E = L0.n_expert, K = L0.top_k, n = L0.d_model, ff = L0.d_ff;
    if (E < 1 || E > 1024 || K < 1 || K > 32 || K > E) return set_error(kErrShape, "moe_stack: E=%d K=%d", E, K);
    if (L0.stride < expert_bytes(n, ff)) return set_error(kErrShape, "moe_stack: stride %zu < blob", L0.stride);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t lw = frt_moe_layer_workspace_bytes(&L0, 1);
    float* buf[2] = {reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + lw),
                     reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + lw + up256(size_t(n) * 4))};
    constexpr int kChunk = 64;   // layers of one persistent launch
    const float* cur = x;
    bool dense = false;   // a dense shared expert: layer by layer (the persistent kernels take the Q2_0 blob)
    for (int l = 0; l < n_layer; ++l) dense = dense || layers[l].shared_dense;
    if (!dense && g_dec1_on && dec2_support(E, K, n, ff, 2)) {
        const LayerWs w = layer_carve(ws, L0, 1, ws_bytes);
        for (int l0 = 0, c = 0; l0 < n_layer; l0 += kChunk, ++c) {
            const int nl = n_layer - l0 < kChunk ? n_layer - l0 : kChunk;
            float* dst = l0 + nl == n_layer ? out : buf[c % 2];
            if (int rc = dec2_stack(layers + l0, nl, cur, dst, ids ? ids + size_t(l0) * K : nullptr,
                                    wts ? wts + size_t(l0) * K : nullptr, w.sync, s))
                return rc;
            cur = dst;
        }
        return kOk;
    }
    if (!dense && g_dec1_on && dec1_support(E, K, n, ff) == 2) {
        const LayerWs w = layer_carve(ws, L0, 1, ws_bytes);
        for (int l0 = 0, c = 0; l0 < n_layer; l0 += kChunk, ++c) {
            const int nl = n_layer - l0 < kChunk ? n_layer - l0 : kChunk;
            float* dst = l0 + nl == n_layer ? out : buf[c % 2];
            if (int rc = dec1_stack(layers + l0, nl, cur, dst, ids ? ids + size_t(l0) * K : nullptr,
                                    wts ? wts + size_t(l0) * K : nullptr, w.sync, s))
                return rc;
            cur = dst;
        }
        return kOk;
    }
    for (int l = 0; l < n_layer; ++l) {   // layer by layer
        float* dst = l + 1 == n_layer ? out : buf[l % 2];
        if (int rc = frt_moe_layer_forward(&layers[l], cur, 1, cur, dst, ids ? ids + size_t(l) * K : nullptr,
                                           wts ? wts + size_t(l) * K : nullptr, nullptr, ws, lw, stream))
            return rc;
        cur = dst;
    }
    return kOk;
}

int frt_set_option(const char* name, int64_t value) {
    if (!name) return set_error(kErrNull, "set_option: null name");
    if (!std::strcmp(name, "decode_fused")) {
        g_dec1_on = value ? 1 : 0;
        return kOk;
    }
    if (!std::strcmp(name, "decode_stamps")) {   // (a device buffer of 64 x 12 x 1024 words, or 0)
        g_dec2_stamps = reinterpret_cast<uint64_t*>(uintptr_t(value));
        return kOk;
    }
    if (!std::strcmp(name, "route_waves")) {   // (8: all waves of the persistent kernels route; 1: one)
        if (value != 1 && value != 8) return set_error(kErrShape, "set_option: route_waves %lld (1 or 8)", (long long)value);
        g_route8 = value == 8 ? 1 : 0;
        return kOk;
    }
    if (!std::strcmp(name, "decode_xcd")) {
        g_dec2_on = value ? 1 : 0;
        return kOk;
    }
    if (!std::strcmp(name, "decode_grid")) {
        if (value < 0 || value > 1024) return set_error(kErrShape, "set_option: decode_grid %lld", (long long)value);
        g_dec1_grid_cap = int(value);
        return kOk;
    }
    if (!std::strcmp(name, "window_min_t")) {   // (2 .. 9; 9: no window path)
        if (value < 2 || value > 9) return set_error(kErrShape, "set_option: window_min_t %lld", (long long)value);
        g_window_min_t = int(value);
        return kOk;
    }
    if (!std::strcmp(name, "router_mfma")) {
        g_router_mfma = value ? 1 : 0;
        return kOk;
    }
    if (!std::strcmp(name, "decode_window_persistent")) {   // 0: windows of 2-4 tokens take the four-launch path
        g_decw_on = value ? 1 : 0;
        return kOk;
    }
    if (!std::strcmp(name, "sync_ticks")) {
        if (value < 0) return set_error(kErrShape, "set_option: sync_ticks < 0");
        g_dec1_ticks = uint64_t(value);
        return kOk;
    }
    return set_error(kErrShape, "set_option: unknown option '%s'", name);
}

int frt_moe_layer_sync_error(void* ws, void* stream) {
    if (!ws) return set_error(kErrNull, "moe_layer_sync_error: null workspace");
    uint32_t err = 0;
    if (int rc = dec1_status(ws, static_cast<hipStream_t>(stream), &err)) return rc;
    return err ? 1 : 0;
}

int frt_moe_layer_forward_ex(const frt_moe_layer* L, const float* x, int T, const float* resid, float* out,
                             int32_t* ids, float* wts, uint32_t* counts, uint32_t* tail_counts, int tail_from,
                             float* probs, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = frt_moe_layer_forward(L, x, T, resid, out, ids, wts, counts, ws, ws_bytes, stream)) return rc;
    if (!tail_counts && !probs) return kOk;
    const int E = L->n_expert, K = L->top_k, n = L->d_model, ff = L->d_ff;
    const LayerWs w = layer_carve(ws, *L, T, ws_bytes);
    const float* lg = w.logits;
    int ls = 1;
    if (T == 1 && g_dec1_on && !L->shared_dense && (dec2_support(E, K, n, ff, 1) || dec1_support(E, K, n, ff) >= 1))
        lg = dec1_logits(w.sync, &ls);   // the persistent call's (both kernels keep them in the same words)
    return layer_trace(lg, ls, ids ? ids : w.ids, T, E, K, tail_counts, tail_from, probs, static_cast<hipStream_t>(stream));
}

int frt_gen_experts(uint64_t seed, int cfg, int layer, int e0, int count, int tensor_base, int n, int ff, float sd,
                    uint8_t* dst, size_t stride, void* stream) {
    if (!dst) return set_error(kErrNull, "gen_experts: null");
    return gen_experts(seed, cfg, layer, e0, count, tensor_base, n, ff, sd, dst, stride, static_cast<hipStream_t>(stream));
}
int frt_gen_normal(uint64_t seed, int cfg, int layer, int tensor, float sd, float* dst, size_t count, int round_bf16,
                   void* stream) {
    if (!dst) return set_error(kErrNull, "gen_normal: null");
    return gen_normal(seed, cfg, layer, tensor, sd, dst, count, round_bf16, static_cast<hipStream_t>(stream));
}
int frt_gen_correlated(uint64_t seed, int cfg, int layer, int tensor0, int T, int n, float rho, float* dst, void* stream) {
    if (!dst || T < 1) return set_error(kErrNull, "gen_correlated: null");
    return gen_correlated(seed, cfg, layer, tensor0, T, n, rho, dst, static_cast<hipStream_t>(stream));
}
void frt_gen_zipf_bias(uint64_t seed, int cfg, int layer, int E, float s, float alpha, float* host_bias) {
    gen_zipf_bias(seed, cfg, layer, E, s, alpha, host_bias);
}

}  // extern "C"
