// C++ client of the flashrt_moe.hpp mirror, written the way the reference's own tests call its
// entry points (tests/test_route_topk.cpp:22-69, tests/test_moe_q2.cpp:97-153).
//   test_shim --host   size queries and error behaviour (no device work)
//   test_shim --gpu    moe_route_topk on the test_route_topk recipe (T 16384, E 512, K 10,
//                      quarter-integer logits with many exact ties) against std::stable_sort and a
//                      double softmax; arena round trip.
// Prints "all passed" and exits 0 on success.
#include "flashrt_moe.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <vector>

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
    check(q2_0::expert_bytes(2048, 512) == 884736, "expert_bytes(2048, 512) == 884736");
    check(q2_0::expert_bytes(2560, 640) == 1382400, "expert_bytes(2560, 640) == 1382400");
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
    ExpertArena a = arena_alloc(2, 3, q2_0::expert_bytes(256, 128));
    check(a.base() != nullptr && a.stride % 4096 == 0 && a.total_bytes() == size_t(6) * a.stride, "arena_alloc");
    std::vector<uint8_t> blob(a.blob_bytes), back(a.blob_bytes);
    for (size_t i = 0; i < blob.size(); ++i) blob[i] = uint8_t(splitmix(s));
    arena_upload(a, 1, 2, blob.data(), st);
    HIP_OK(hipStreamSynchronize(st));
    HIP_OK(hipMemcpy(back.data(), a.blob(1, 2), back.size(), hipMemcpyDeviceToHost));
    check(blob == back && a.blob(1, 2) == a.base() + 5 * a.stride, "arena upload round trip and blob(l, e) address");
    arena_free(a);
    HIP_OK(hipStreamDestroy(st));
    HIP_OK(hipFree(d_lg));
    HIP_OK(hipFree(d_w));
    HIP_OK(hipFree(d_ids));
    HIP_OK(hipFree(d_cnt));
}

}  // namespace

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    host_checks();
    if (gpu) gpu_checks();
    if (g_fail) {
        std::printf("%d FAILED\n", g_fail);
        return 1;
    }
    std::printf("all passed\n");
    return 0;
}
