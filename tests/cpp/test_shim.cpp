// C++ client of the flashrt_moe.hpp mirror, written the way the reference's own tests and engine
// call its entry points (tests/test_route_topk.cpp:22-69, tests/test_moe_q2.cpp:97-153,
// engine/session.cpp:113-117,171-179, tools/fr_bench.cpp:204-213,403-408).
//   test_shim --host   size queries, the host repack, error behaviour (no device work)
//   test_shim --gpu    moe_route_topk on the test_route_topk recipe (T 16384, E 512, K 10,
//                      quarter-integer logits with many exact ties) against std::stable_sort and a
//                      double softmax; arena round trip; the engine's set-up statements, verbatim,
//                      over a synthetic GGUF expert slab file (load_experts, arena_register, the
//                      cache / doorbell shims) and layer calls through moe_block_fast and
//                      moe_block_stream with counts, tail counts and a MoeTrace.
// Prints "all passed" and exits 0 on success.
#include "flashrt_moe.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <numeric>
#include <string>
#include <vector>

#include <unistd.h>

namespace {

int g_fail = 0;
void check(bool ok, const char* what) {
    std::printf("%-60s %s\n", what, ok ? "ok" : "FAILED");
    if (!ok) ++g_fail;
}

template <typename F>
bool throws(F&& f) {
    try {
        f();
    } catch (const std::runtime_error&) {
        return true;
    }
    return false;
}

#define HIP_OK(x)                                                                   \
    do {                                                                            \
        if ((x) != hipSuccess) {                                                    \
            std::printf("HIP error at %s:%d: %s\n", __FILE__, __LINE__, #x);        \
            std::exit(2);                                                           \
        }                                                                           \
    } while (0)

uint64_t splitmix(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void host_checks() {
    using namespace flashrt;
    check(q2_0::mat_bytes(512, 2048) == 294912, "mat_bytes(512, 2048) == 294912");
    check(q2_0::expert_bytes({2048, 512}) == 884736, "expert_bytes({2048, 512}) == 884736");
    check(q2_0::expert_bytes({2560, 640}) == 1382400, "expert_bytes({2560, 640}) == 1382400");
    {   // the planar repack of one block, element by element (tests/test_q2_0.cpp:74-86's check)
        uint8_t in[18], out[18];
        uint64_t s = 5;
        for (auto& b : in) b = uint8_t(splitmix(s));
        q2_0::repack(in, 1, 64, out);
        bool ok = out[16] == in[0] && out[17] == in[1];
        for (int j = 0; j < 64; ++j) ok &= ((in[2 + j / 4] >> (2 * (j % 4))) & 3) == ((out[j % 16] >> (2 * (j / 16))) & 3);
        check(ok, "q2_0::repack places element j at byte j % 16, bits 2 (j / 16)");
    }
    check(throws([] { uint8_t b[18]; q2_0::repack(b, 1, 32, b); }), "q2_0::repack cols % 64 != 0 throws");
    check(moe_q2::workspace_bytes(2048, 10, 2048, 512, 512) > 0, "moe_q2::workspace_bytes > 0");
    check(throws([] { qwen4exp::moe_route_topk(nullptr, nullptr, 1, 512, 0, nullptr, nullptr, nullptr); }),
          "moe_route_topk k = 0 throws");
    check(throws([] { qwen4exp::moe_route_topk(nullptr, nullptr, 1, 2048, 10, nullptr, nullptr, nullptr); }),
          "moe_route_topk E > 1024 throws");
    check(throws([] {
              moe_q2::run(nullptr, 0, 512, 2048, 512, nullptr, nullptr, 16, 10, nullptr, nullptr, 0, nullptr, true);
          }),
          "moe_q2::run block64 throws");
    check(throws([] {
              moe_q2::run(nullptr, 0, 512, 2000, 512, nullptr, nullptr, 16, 10, nullptr, nullptr, 0, nullptr);
          }),
          "moe_q2::run n % 256 != 0 throws");
}

void gpu_checks() {
    using namespace flashrt;
    const int T = 16384, E = 512, K = 10;
    std::vector<float> lg(size_t(T) * E);
    uint64_t s = 9;
    for (auto& v : lg) {   // round(N(0, 2) * 4) / 4 via Box-Muller in double
        const double u1 = (double(splitmix(s) >> 11) + 0.5) * 0x1p-53, u2 = double(splitmix(s) >> 11) * 0x1p-53;
        const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
        v = float(std::round(z * 2.0 * 4.0) / 4.0);
    }
    float *d_lg, *d_w;
    int32_t* d_ids;
    uint32_t* d_cnt;
    HIP_OK(hipMalloc(&d_lg, lg.size() * 4));
    HIP_OK(hipMalloc(&d_w, size_t(T) * K * 4));
    HIP_OK(hipMalloc(&d_ids, size_t(T) * K * 4));
    HIP_OK(hipMalloc(&d_cnt, E * 4));
    HIP_OK(hipMemcpy(d_lg, lg.data(), lg.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemset(d_cnt, 0, E * 4));
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    qwen4exp::moe_route_topk(st, d_lg, T, E, K, d_ids, d_w, d_cnt);
    HIP_OK(hipStreamSynchronize(st));
    std::vector<int32_t> ids(size_t(T) * K);
    std::vector<float> w(size_t(T) * K);
    std::vector<uint32_t> cnt(E);
    HIP_OK(hipMemcpy(ids.data(), d_ids, ids.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(w.data(), d_w, w.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(cnt.data(), d_cnt, cnt.size() * 4, hipMemcpyDeviceToHost));
    bool ids_ok = true, cnt_ok = true;
    double worst = 0;
    std::vector<uint32_t> want_cnt(E, 0);
    std::vector<int> idx(E);
    for (int t = 0; t < T; ++t) {
        const float* l = &lg[size_t(t) * E];
        std::iota(idx.begin(), idx.end(), 0);
        std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return l[a] > l[b]; });
        double mx = l[idx[0]], sum_top = 0;
        for (int k = 0; k < K; ++k) sum_top += std::exp(double(l[idx[k]]) - mx);
        for (int k = 0; k < K; ++k) {
            ids_ok &= ids[size_t(t) * K + k] == idx[k];
            ++want_cnt[idx[k]];
            const double ref = std::exp(double(l[idx[k]]) - mx) / sum_top;
            worst = std::max(worst, std::fabs(w[size_t(t) * K + k] - ref) / ref);
        }
    }
    for (int e = 0; e < E; ++e) cnt_ok &= cnt[e] == want_cnt[e];
    check(ids_ok, "route_topk ids == stable sort (ties to the lower id)");
    check(cnt_ok, "route_topk counts exact");
    std::printf("route_topk weights: max relative error %.3g\n", worst);
    check(worst <= 1e-6, "route_topk weights within 1e-6 relative");

    // arena: upload one blob, read it back
    ExpertArena a = arena_alloc(2, 3, q2_0::expert_bytes({256, 128}), PageMode::Default, 0);
    check(a.buf.ptr != nullptr && a.stride % 4096 == 0 && a.total_bytes() == size_t(6) * a.stride, "arena_alloc");
    std::vector<uint8_t> blob(a.blob_bytes), back(a.blob_bytes);
    for (size_t i = 0; i < blob.size(); ++i) blob[i] = uint8_t(splitmix(s));
    arena_upload(a, 1, 2, blob.data(), st);
    HIP_OK(hipStreamSynchronize(st));
    HIP_OK(hipMemcpy(back.data(), a.blob(1, 2), back.size(), hipMemcpyDeviceToHost));
    check(blob == back && a.blob(1, 2) == static_cast<uint8_t*>(a.buf.ptr) + 5 * a.stride,
          "arena upload round trip and blob(l, e) address");
    arena_free(a);
    HIP_OK(hipStreamDestroy(st));
    HIP_OK(hipFree(d_lg));
    HIP_OK(hipFree(d_w));
    HIP_OK(hipFree(d_ids));
    HIP_OK(hipFree(d_cnt));
}

}  // namespace

// ---- stand-ins for the engine's own types (not part of the MoE path): just the members the
// reference's set-up statements below touch
namespace flashrt {
class CpuPool {
  public:
    CpuPool(int workers, const std::vector<int>& cpus) : workers_(workers), cpus_(cpus) {}
    void set_spin_us(int us) { spin_us_ = us; }
    int workers_, spin_us_ = 0;
    std::vector<int> cpus_;
};
std::vector<int> physical_cpus() { return {0, 1, 2, 3}; }
bool pin_current_thread(int) { return true; }
struct GgufTensor {
    std::string name;
    int shard = 0;
    uint64_t file_offset = 0;
};
struct Gguf {
    std::vector<std::string> shards;
    std::vector<GgufTensor> tensors;
    const GgufTensor* tensor(const std::string& name) const {
        for (const auto& x : tensors)
            if (x.name == name) return &x;
        return nullptr;
    }
};
namespace qwen4exp {
struct Spec {
    int n_layer, n_expert, n_expert_used, d_model, d_ff_expert;
};
struct BlockCtx {
    hipStream_t stream;
};
struct Forward {
    hipStream_t s = nullptr;
    bool graphs = false;
    ExpertCache* cache = nullptr;
    MoeFastHost* host = nullptr;
    hipStream_t stream() const { return s; }
    void set_graphs(bool on) { graphs = on; }
    void set_fast_moe(ExpertCache* c, MoeFastHost* h) {
        cache = c;
        host = h;
    }
};
struct SessionOptions {
    int workers = 3;
};
using Clock = std::chrono::steady_clock;

// A small model's expert slabs in ggml Q2_0 layout written to `path`: per layer gate, up, down
// slabs of n_expert matrices each, 4 KiB apart like GGUF tensor data; fills g.
void write_slabs(const Spec& s, const std::string& path, Gguf& g, std::vector<std::vector<uint8_t>>& slabs) {
    std::FILE* f = std::fopen(path.c_str(), "wb");
    uint64_t off = 4096, seed = 77;
    const size_t mb[3] = {q2_0::mat_bytes(s.d_ff_expert, s.d_model), q2_0::mat_bytes(s.d_ff_expert, s.d_model),
                          q2_0::mat_bytes(s.d_model, s.d_ff_expert)};
    const char* names[3] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    std::vector<uint8_t> zero(4096, 0);
    std::fwrite(zero.data(), 1, 4096, f);
    g.shards = {path};
    for (int l = 0; l < s.n_layer; ++l)
        for (int k = 0; k < 3; ++k) {
            std::vector<uint8_t> sl(mb[k] * s.n_expert);
            for (size_t i = 0; i < sl.size(); i += 18) {   // blocks: fp16 scale in [0.005, 0.02), random codes
                const float d = 0.005f + 0.015f * float(splitmix(seed) >> 40) / float(1 << 24);
                const _Float16 h = _Float16(d);
                std::memcpy(&sl[i], &h, 2);
                for (int j = 2; j < 18; ++j) sl[i + j] = uint8_t(splitmix(seed));
            }
            g.tensors.push_back({"blk." + std::to_string(l) + "." + names[k] + ".weight", 0, off});
            std::fwrite(sl.data(), 1, sl.size(), f);
            off += sl.size();
            const size_t pad = (4096 - off % 4096) % 4096;
            std::fwrite(zero.data(), 1, pad, f);
            off += pad;
            slabs.push_back(std::move(sl));
        }
    std::fclose(f);
}

// engine/session.cpp:113-117 and :171-179, statements as they are there
void session_setup(const Spec& s, const Gguf& g, ExpertArena& arena, ExpertCache& cache, MoeFastHost& host,
                   std::unique_ptr<CpuPool>& pool, std::unique_ptr<Forward>& fwd, std::vector<int>& cpus,
                   const SessionOptions& o, int W) {
    auto stage = [](const char* what) { std::printf("stage: %s\n", what); };
    arena = arena_alloc(s.n_layer, s.n_expert, q2_0::expert_bytes({s.d_model, s.d_ff_expert}), PageMode::THP, 0);
    if (!arena.buf.ptr) throw std::runtime_error("expert arena allocation failed");
    load_experts(g, s, arena, 12);
    arena_register(arena);   // now, not in the first long prompt's prefill
    stage("experts read into the host arena and registered");
    cpus = physical_cpus();
    pool = std::make_unique<CpuPool>(o.workers, cpus);
    fwd = std::make_unique<Forward>();
    size_t free_b = size_t(1) << 30, keep = 0, eb = q2_0::expert_bytes({s.d_model, s.d_ff_expert});
    cache = alloc_expert_cache(s, int((free_b - keep) / eb));
    host = alloc_moe_fast_host(s, W);
    host.arena = &arena;
    host.pool = pool.get();
    start_doorbell(s, host, cpus[0]);                             // the miss server takes cpus[0]
    pin_current_thread(cpus[size_t(o.workers) % cpus.size()]);    // this (the enqueue) thread moves off it
    pool->set_spin_us(2000);
    fwd->set_graphs(true);
    fwd->set_fast_moe(&cache, &host);
}

// tools/fr_bench.cpp:204-213 and :403-408, statements as they are there
int bench_setup(const Spec& s, const Gguf& g, int workers, int slots, int spec_k, Forward& fwd,
                const std::vector<std::pair<int, int>>& order, ExpertCache& cache, MoeFastHost& host,
                ExpertArena& arena_out) {
    ExpertArena arena = arena_alloc(s.n_layer, s.n_expert, q2_0::expert_bytes({s.d_model, s.d_ff_expert}), PageMode::THP, 0);
    if (!arena.buf.ptr) { std::fprintf(stderr, "arena allocation failed\n"); return 1; }
    load_experts(g, s, arena, 12);
    {
        const auto tr = Clock::now();
        arena_register(arena);   // at load, outside the timed prefill
        std::printf("expert arena registered in %.1f s\n", std::chrono::duration<double>(Clock::now() - tr).count());
    }
    const std::vector<int> cpus = physical_cpus();
    CpuPool pool(workers, cpus);   // pins this thread to cpus[0]
    const auto tf = Clock::now();
    const double free_b = double(size_t(1) << 30);
        cache = alloc_expert_cache(s, slots);
        expert_cache_fill(s, cache, arena, order, fwd.stream());
        std::printf("expert cache: %d slots (%.1f%% of experts), filled in %.1f s from %.0f MiB free\n", slots,
                    100.0 * slots / (s.n_layer * s.n_expert), std::chrono::duration<double>(Clock::now() - tf).count(),
                    free_b / 1048576.0);
        host = alloc_moe_fast_host(s, spec_k + 1);
        host.arena = &arena;
        host.pool = &pool;
    host.pool = nullptr;   // the stand-in pool ends here
    arena_out = arena;
    return 0;
}
}  // namespace qwen4exp
}  // namespace flashrt

namespace {

void engine_checks() {
    using namespace flashrt;
    using namespace flashrt::qwen4exp;
    const Spec s{2, 8, 2, 1024, 256};
    const std::string path = "/tmp/frt_test_slabs_" + std::to_string(::getpid()) + ".gguf";
    Gguf g;
    std::vector<std::vector<uint8_t>> slabs;
    write_slabs(s, path, g, slabs);
    ExpertArena arena;
    ExpertCache cache;
    MoeFastHost host;
    std::unique_ptr<CpuPool> pool;
    std::unique_ptr<Forward> fwd;
    std::vector<int> cpus;
    SessionOptions o;
    bool ok = true;
    try {
        session_setup(s, g, arena, cache, host, pool, fwd, cpus, o, 1);
    } catch (const std::exception& e) {
        std::printf("session set-up threw: %s\n", e.what());
        ok = false;
    }
    check(ok && arena.buf.ptr && host.doorbell && fwd->cache == &cache && pool->spin_us_ == 2000,
          "session.cpp:113-117,171-179 set-up runs");
    // the loaded blobs equal the host repack of the same ggml bytes
    const q2_0::ExpertShape shape{s.d_model, s.d_ff_expert};
    const size_t mb[3] = {q2_0::mat_bytes(s.d_ff_expert, s.d_model), q2_0::mat_bytes(s.d_ff_expert, s.d_model),
                          q2_0::mat_bytes(s.d_model, s.d_ff_expert)};
    std::vector<uint8_t> want(arena.blob_bytes), got(arena.blob_bytes);
    bool same = ok;
    for (int l = 0; l < s.n_layer && same; ++l)
        for (int e = 0; e < s.n_expert && same; ++e) {
            q2_0::repack_expert(&slabs[3 * l][e * mb[0]], &slabs[3 * l + 1][e * mb[1]], &slabs[3 * l + 2][e * mb[2]], shape,
                                want.data());
            HIP_OK(hipMemcpy(got.data(), arena.blob(l, e), got.size(), hipMemcpyDeviceToHost));
            same &= want == got;
        }
    check(same, "load_experts: every arena blob == repack_expert of its slab bytes");
    check(arena_register(arena) == arena.buf.ptr, "arena_register returns the device base");
    check(cache.n_slots == s.n_layer * s.n_expert && cache.table[size_t(1) * s.n_expert + 3] == s.n_expert + 3,
          "alloc_expert_cache: the identity table");
    bool missing = throws([&] {
        Gguf bad = g;
        bad.tensors.pop_back();
        ExpertArena a2 = arena_alloc(s.n_layer, s.n_expert, q2_0::expert_bytes({s.d_model, s.d_ff_expert}), PageMode::THP, 0);
        try {
            load_experts(bad, s, a2, 2);
        } catch (...) {
            arena_free(a2);
            throw;
        }
        arena_free(a2);
    });
    check(missing, "load_experts: a missing slab tensor throws");

    // fr_bench.cpp:204-213, 403-408
    ExpertCache cache2;
    MoeFastHost host2;
    ExpertArena arena2;
    std::vector<std::pair<int, int>> order = {{0, 1}, {1, 0}};
    const int rc = bench_setup(s, g, 3, 6, 1, *fwd, order, cache2, host2, arena2);
    check(rc == 0 && cache2.slots == arena2.buf.ptr && cache2.slot_bytes == arena2.stride && host2.max_window == 2,
          "fr_bench.cpp:204-213,403-408 set-up runs");

    // layer calls: moe_block_fast (T = 1) and moe_block_stream (T = 64) on layer 1 of the arena
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    const int n = s.d_model, E = s.n_expert, K = s.n_expert_used, T = 64;
    uint64_t seed = 3;
    auto dev_normal = [&](size_t cnt, float sd) {
        std::vector<float> v(cnt);
        for (auto& x : v) {
            const double u1 = (double(splitmix(seed) >> 11) + 0.5) * 0x1p-53, u2 = double(splitmix(seed) >> 11) * 0x1p-53;
            x = float(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2) * sd);
        }
        float* d;
        HIP_OK(hipMalloc(&d, cnt * 4));
        HIP_OK(hipMemcpy(d, v.data(), cnt * 4, hipMemcpyHostToDevice));
        return d;
    };
    float* router = dev_normal(size_t(E) * n, 0.02f);
    float* gate = dev_normal(n, 0.02f);
    float* x = dev_normal(size_t(T) * n, 1.0f);
    float *out_a, *out_b, *probs;
    int32_t* ids;
    uint32_t *counts, *tail;
    HIP_OK(hipMalloc(&out_a, size_t(T) * n * 4));
    HIP_OK(hipMalloc(&out_b, size_t(T) * n * 4));
    HIP_OK(hipMalloc(&probs, size_t(T) * K * 4));
    HIP_OK(hipMalloc(&ids, size_t(T) * K * 4));
    HIP_OK(hipMalloc(&counts, E * 4));
    HIP_OK(hipMalloc(&tail, E * 4));
    HIP_OK(hipMemset(counts, 0, E * 4));
    HIP_OK(hipMemset(tail, 0, E * 4));
    const MoeLayer L1(arena.blob(1, 0), arena.stride, E, arena.blob(0, 7), router, nullptr, gate, n, s.d_ff_expert, K);
    host.set_layer(1, L1);
    const BlockCtx c{st};
    moe_block_fast(c, 1, x, cache, host, out_a, 1);
    void* ws;
    const size_t wsb = L1.workspace_bytes(T);
    HIP_OK(hipMalloc(&ws, wsb));
    L1.forward(x, 1, out_b, ws, wsb, st);
    std::vector<float> a1(n), b1(n);
    HIP_OK(hipStreamSynchronize(st));
    HIP_OK(hipMemcpy(a1.data(), out_a, n * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(b1.data(), out_b, n * 4, hipMemcpyDeviceToHost));
    check(a1 == b1 && std::isfinite(a1[0]), "moe_block_fast == MoeLayer::forward (T = 1)");
    ExpertStream* es = create_expert_stream(s, arena, T);
    es->set_layer(1, L1);
    expert_stream_prefetch(es, 1);
    moe_block_stream(c, 1, x, T, *es, out_a, counts, tail, 48);
    L1.forward(x, T, out_b, ws, wsb, st);
    std::vector<float> at(size_t(T) * n), bt(size_t(T) * n);
    std::vector<uint32_t> hc(E), ht(E);
    HIP_OK(hipStreamSynchronize(st));
    HIP_OK(hipMemcpy(at.data(), out_a, at.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(bt.data(), out_b, bt.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hc.data(), counts, E * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(ht.data(), tail, E * 4, hipMemcpyDeviceToHost));
    const long sc = std::accumulate(hc.begin(), hc.end(), 0L), stl = std::accumulate(ht.begin(), ht.end(), 0L);
    check(at == bt, "moe_block_stream == MoeLayer::forward (T = 64)");
    check(sc == long(T) * K && stl == long(T - 48) * K, "moe_block_stream counts every selection, tail_counts those of t >= 48");
    check(expert_stream_bytes(es) >= expert_stream_bytes_for(s, arena, T), "expert_stream_bytes");
    destroy_expert_stream(es);
    // MoeTrace: ids and probabilities before renormalisation; the weights are their renormalisation
    MoeTrace tr;
    float* wts;
    HIP_OK(hipMalloc(&wts, size_t(T) * K * 4));
    L1.forward_traced(x, T, out_a, ws, wsb, st, tr, ids, probs);
    L1.forward(x, T, out_b, ws, wsb, st, nullptr, nullptr, wts);
    std::vector<float> wv(size_t(T) * K);
    HIP_OK(hipStreamSynchronize(st));
    HIP_OK(hipMemcpy(wv.data(), wts, wv.size() * 4, hipMemcpyDeviceToHost));
    double worst = 0;
    bool pr_ok = true;
    for (int t = 0; t < T; ++t) {
        double sp = 0;
        for (int k = 0; k < K; ++k) sp += tr.probs[size_t(t) * K + k];
        pr_ok &= sp > 0 && sp <= 1.0 + 1e-6;
        for (int k = 0; k < K; ++k) {
            const double w = tr.probs[size_t(t) * K + k] / sp;
            worst = std::max(worst, std::fabs(w - wv[size_t(t) * K + k]) / w);
            pr_ok &= tr.topk[size_t(t) * K + k] >= 0 && tr.topk[size_t(t) * K + k] < E;
        }
    }
    check(pr_ok && worst < 1e-5, "MoeTrace: probs in (0, 1], their renormalisation == the weights");
    doorbell_begin_token(host, 1);
    doorbell_end_token(host, s);
    CacheManager* mgr = create_cache_manager(s, cache, arena, CachePolicyConfig{}, std::vector<uint32_t>(16, 0));
    cache_manager_step(mgr, host, st);
    check(!doorbell_failed(host) && cache_check(cache, mgr).host_resident == cache.n_slots &&
              cache_manager_stats(mgr).swaps == 0,
          "doorbell / cache-manager shims");
    destroy_cache_manager(mgr);
    for (void* p : {(void*)router, (void*)gate, (void*)x, (void*)out_a, (void*)out_b, (void*)probs, (void*)ids,
                    (void*)counts, (void*)tail, ws, (void*)wts})
        HIP_OK(hipFree(p));
    HIP_OK(hipStreamDestroy(st));
    free_moe_fast_host(host);
    free_moe_fast_host(host2);
    free_expert_cache(cache);
    free_expert_cache(cache2);
    arena_free(arena2);
    arena_free(arena);
    std::remove(path.c_str());
}

}  // namespace

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    host_checks();
    if (gpu) {
        gpu_checks();
        engine_checks();
    }
    if (g_fail) {
        std::printf("%d FAILED\n", g_fail);
        return 1;
    }
    std::printf("all passed\n");
    return 0;
}
