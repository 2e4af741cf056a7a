// Pieces shared by the persistent single-token kernels (decode1.hip, decode2.hip): the sync region's
// header (error word, epoch cells), the epoch-tagged words their in-kernel joins use, and the
// bounded wait for such words.
//
// A tagged word is (tag << 32) | payload, stored and loaded as one 8-byte access. tag = f(epoch):
// each call's epoch exceeds every epoch stored before it in the region (the largest cell + 1), so a
// word is current exactly when its tag matches, and no flag, fence or counter is needed.
//   - Words read on other XCDs are stored at agent scope (written through this XCD's L2).
//   - Words read only on the writer's own XCD are stored at workgroup scope: they stay in the XCD's
//     L2, which every CU of the XCD shares (workgroup b of a launch runs on XCD b mod 8).
//   - Every poll is an agent-scope load: it bypasses the CU's L1 (a workgroup-scope load can be
//     served by a stale L1 line) and sees both kinds of word.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frt {

constexpr int kMaxGrid = 1024;
constexpr int kMaxStack = 64;   // layers of one stack call (their table travels in the kernel arguments)
constexpr uint32_t kErrMagic = 0x5E7C0DE5u;   // upper half of a set error word (garbage rarely matches)
struct Dec1Sync {
    uint64_t err;                // (kErrMagic << 32) | epoch of a call whose wait ran out of time; else anything
    uint32_t pad[62];
    uint32_t epoch[kMaxGrid];    // per workgroup: its last call's epoch
};

// The sync region at the front of every layer workspace: this header, the logits' tagged words
// (any stride up to 16 words), then either kernel's other words.
constexpr size_t kSyncHead = (sizeof(Dec1Sync) + 255) / 256 * 256;
constexpr size_t kSyncLg = size_t(1024 + 1 + 31) / 32 * 32 * 8 * 16;
// decode2.hip, per XCD: the relayed logits, the h values, the down partials, the next layer's input
constexpr int kD2LglWords = 1056;
constexpr int kD2HlWords = 4096;
constexpr int kD2XWords = 4096;
constexpr size_t kD2Tail = size_t(8) * (kD2LglWords + kD2HlWords + 2 * kD2XWords) * 8;

struct Dec1Layer {
    const float* W;        // [E][n] router
    const float* bias;     // [E] or null
    const float* gate_w;   // [n] shared-expert gate
    const uint8_t* arena;  // routed expert 0 of the layer
    const uint8_t* shared;
};

namespace {

constexpr int kNTP = 512;   // threads per workgroup of the persistent kernels

__device__ __forceinline__ uint32_t sync_tag(uint32_t e) { return (e * 0x9E3779B1u) ^ 0x7F4A7C15u; }
// a word for other XCDs
__device__ __forceinline__ void pub(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, (uint64_t(tag) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// a word for this XCD only
__device__ __forceinline__ void pub_local(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, (uint64_t(tag) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint64_t peek(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits for the tagged words i = threadIdx.x + k kNTP < count (k < MAXK), word i at base + i STRIDE,
// and hands each payload to put(i, payload). Out of time: sets the error word (err_val) and the
// host-visible flag (if any) and hands over what it last read.
template <int MAXK, int NT = kNTP, class A, class F>
__device__ __forceinline__ void wait_words_at(A addr, int count, uint32_t tag, uint64_t deadline, uint64_t* err,
                                              uint64_t err_val, uint32_t* host_err, F put, int t0 = 0);
template <int MAXK, int STRIDE = 1, class F>
__device__ __forceinline__ void wait_words(const uint64_t* base, int count, uint32_t tag, uint64_t deadline,
                                           uint64_t* err, uint64_t err_val, uint32_t* host_err, F put) {
    wait_words_at<MAXK>([&](int i) { return base + size_t(i) * STRIDE; }, count, tag, deadline, err, err_val,
                        host_err, put);
}
// The same for word i at addr(i), waited for by the NT threads t0 .. t0 + NT - 1 (thread t0 + q takes
// words q + k NT).
template <int MAXK, int NT, class A, class F>
__device__ __forceinline__ void wait_words_at(A addr, int count, uint32_t tag, uint64_t deadline, uint64_t* err,
                                              uint64_t err_val, uint32_t* host_err, F put, int t0) {
    const int q = int(threadIdx.x) - t0;
    uint32_t pend = 0;
#pragma unroll
    for (int k = 0; k < MAXK; ++k)
        if (q + k * NT < count) pend |= 1u << k;
    while (pend) {
        uint64_t v[MAXK];
#pragma unroll
        for (int k = 0; k < MAXK; ++k) v[k] = ((pend >> k) & 1u) ? peek(addr(q + k * NT)) : 0ull;
#pragma unroll
        for (int k = 0; k < MAXK; ++k)
            if (((pend >> k) & 1u) && uint32_t(v[k] >> 32) == tag) {
                put(q + k * NT, uint32_t(v[k]));
                pend &= ~(1u << k);
            }
        // a short back-off between polls: the polls of 256 workgroups share the fabric with the weight
        // loads (measured per token: none 710 us, 2 x 64 cycles 707.5, 8 x 64 cycles 725; two polls
        // in flight instead of one: 838)
        if (pend) __builtin_amdgcn_s_sleep(2);
        if (pend && wall_clock64() > deadline) {
            __hip_atomic_store(err, err_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (host_err) __hip_atomic_store(host_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
            for (int k = 0; k < MAXK; ++k)
                if ((pend >> k) & 1u) put(q + k * NT, uint32_t(v[k]));
            break;
        }
    }
}

}  // namespace

// host side (decode1.hip): the host-visible time-out flag of the current device (allocated at the first
// persistent launch unless the caller may not allocate), and the sync region's layout
int host_err_flag(int dev, bool may_alloc, uint32_t** dptr);
extern thread_local bool g_dec1_no_alloc;

}  // namespace frt
