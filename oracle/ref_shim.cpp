// CPU ORACLE — test infrastructure only (see oracle.h).
//
// A C-ABI shim over the reference's own CPU sources (quant/q2_0/*.cpp, core/cpu_pool.cpp,
// core/platform.cpp), compiled where they lie under /root/reference by oracle/Makefile into
// oracle/_ref/libfrref.so. Tests use it to pin the restatement in moe_oracle.cpp; bench.py's
// cpu_baseline leg times its moe_cpu on a CpuPool. No reference source is copied here: this file
// only calls the reference's public API (quant/q2_0/q2_0.hpp, moe_cpu.hpp, core/cpu_pool.hpp).
#include "core/cpu_pool.hpp"
#include "core/fp16.hpp"
#include "core/platform.hpp"
#include "quant/q2_0/moe_cpu.hpp"
#include "quant/q2_0/q2_0.hpp"

#include <cstdint>
#include <cstring>
#include <vector>

using namespace flashrt;
using namespace flashrt::q2_0;

namespace {
struct Q8Buf {
    std::vector<uint8_t> mem;
    Q8Act a;
    Q8Buf(const float* x, int n) : mem(q8_bytes(n) + 64) {
        auto p = (reinterpret_cast<uintptr_t>(mem.data()) + 63) & ~uintptr_t(63);
        a = q8_view(reinterpret_cast<void*>(p), n);
        quantize_q8(x, a);
    }
};
}  // namespace

extern "C" {

int ref_have_avx512() { return have_avx512() ? 1 : 0; }
uint16_t ref_f32_to_f16(float f) { return fp32_to_fp16(f); }
float ref_f16_to_f32(uint16_t h) { return fp16_to_fp32(h); }
size_t ref_expert_bytes(int n, int ff) { return expert_bytes(ExpertShape{n, ff}); }
void ref_repack(const void* ggml, int rows, int cols, void* dst) { repack(ggml, rows, cols, dst); }

// x [n] -> qs [n], d [n/32]
void ref_quantize_q8(const float* x, int n, int8_t* qs, float* d) {
    Q8Buf b(x, n);
    std::memcpy(qs, b.a.qs, size_t(n));
    std::memcpy(d, b.a.d, size_t(n / 32) * 4);
}

// x [ntok][cols] float, quantized inside; use_avx 0: matvec_ref, 1: matvec_avx512
void ref_matvec(const void* w, int rows, int cols, const float* x, int ntok, int r0, int r1, float* y, int ldy,
                int use_avx) {
    const Mat m = mat_view(w, rows, cols);
    std::vector<Q8Buf*> bufs;
    std::vector<Q8Act> a;
    for (int t = 0; t < ntok; ++t) {
        bufs.push_back(new Q8Buf(x + size_t(t) * cols, cols));
        a.push_back(bufs.back()->a);
    }
    if (use_avx) matvec_avx512(m, a.data(), ntok, r0, r1, y, ldy);
    else matvec_ref(m, a.data(), ntok, r0, r1, y, ldy);
    for (auto* b : bufs) delete b;
}

// ggml-layout dot for one row (ggml blocks), x quantized inside
float ref_dot_ggml(const void* ggml_row, const float* x, int cols) {
    Q8Buf b(x, cols);
    return dot_ggml(static_cast<const GgmlBlock*>(ggml_row), b.a);
}

void ref_expert_ffn(const void* blob, int n, int ff, const float* x, int ntok, float* out, int ldo, int use_avx) {
    const Expert e = expert_view(blob, ExpertShape{n, ff});
    std::vector<Q8Buf*> bufs;
    std::vector<Q8Act> a;
    for (int t = 0; t < ntok; ++t) {
        bufs.push_back(new Q8Buf(x + size_t(t) * n, n));
        a.push_back(bufs.back()->a);
    }
    std::vector<uint8_t> scratch(expert_scratch_bytes(ExpertShape{n, ff}));
    expert_ffn(e, a.data(), ntok, out, ldo, scratch.data(), use_avx != 0);
    for (auto* b : bufs) delete b;
}

// A CpuPool pinned to the physical CPUs (as tools/bench_moe_cpu.cpp:77 does), or unpinned.
void* ref_pool_create(int n_workers, int pin) { return new CpuPool(n_workers, pin ? physical_cpus() : std::vector<int>{}); }
// A pool pinned to the given CPUs (the reference's bench pins its pool to physical_cpus(),
// tools/bench_moe_cpu.cpp:76-77; a caller confined to part of the machine passes the physical cores
// it may use, one logical CPU each).
void* ref_pool_create_cpus(int n_workers, const int* cpus, int n_cpus) {
    return new CpuPool(n_workers, std::vector<int>(cpus, cpus + n_cpus));
}
void ref_pool_destroy(void* p) { delete static_cast<CpuPool*>(p); }
int ref_physical_cpus() { return int(physical_cpus().size()); }

// A prepared moe_cpu call: the window's activations quantized once, the Miss list and scratch.
struct RefMoe {
    ExpertShape s;
    std::vector<Q8Buf*> x;
    std::vector<Q8Act> xa;
    std::vector<Miss> miss;
    std::vector<uint8_t> scratch;
};

void* ref_moe_prepare(void* pool, int n, int ff, const uint8_t* const* blobs, const int* ntok, const int* tok,
                      const float* w, int n_miss, const float* x, int T) {
    auto* r = new RefMoe;
    r->s = ExpertShape{n, ff};
    for (int t = 0; t < T; ++t) {
        r->x.push_back(new Q8Buf(x + size_t(t) * n, n));
        r->xa.push_back(r->x.back()->a);
    }
    for (int i = 0; i < n_miss; ++i) {
        Miss m{blobs[i], ntok[i], {}, {}};
        for (int j = 0; j < 4; ++j) {
            m.tok[j] = tok[i * 4 + j];
            m.w[j] = w[i * 4 + j];
        }
        r->miss.push_back(m);
    }
    r->scratch.resize(moe_cpu_scratch_bytes(r->s, n_miss, static_cast<CpuPool*>(pool)->size()) + 64);
    return r;
}

void ref_moe_run(void* pool, void* prep, float* out, int ldo) {
    auto* r = static_cast<RefMoe*>(prep);
    moe_cpu(*static_cast<CpuPool*>(pool), r->s, r->miss.data(), int(r->miss.size()), r->xa.data(), int(r->xa.size()), out,
            ldo, r->scratch.data());
}

void ref_moe_free(void* prep) {
    auto* r = static_cast<RefMoe*>(prep);
    for (auto* b : r->x) delete b;
    delete r;
}

}  // extern "C"
