// Shared definitions of the MI355X (gfx950) MoE library: the planar Q2_0 layout, error
// plumbing for the C ABI, and small wave64 helpers.
//
// Planar Q2_0 (the reference's repacked layout, quant/q2_0/q2_0.hpp:5-15): a rows x cols matrix
// is codes [rows][cols/64][16] followed by fp16 scales [rows][cols/64]; element j of a 64-block is
// in code byte j % 16 at bits 2*(j/16) and decodes to (q - 1) * d. An expert blob is
// gate [ff][n] | up [ff][n] | down [n][ff].
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>

namespace frt {

constexpr int kBlock = 64;   // weights per Q2_0 block
constexpr int kQ8 = 32;      // activations per Q8_0 block
constexpr int kWave = 64;

__host__ __device__ inline size_t mat_bytes(int rows, int cols) { return size_t(rows) * (cols / kBlock) * 18; }
__host__ __device__ inline size_t expert_bytes(int n, int ff) { return 2 * mat_bytes(ff, n) + mat_bytes(n, ff); }

// K order of the prefill GEMM operands within each 256-element stretch (four Q2_0 blocks), perm256.
// MFMA lane group g holds block g of the stretch as one 16-byte code chunk; K-step t (0..7, 32 deep)
// takes from it code dword t / 2, codes 4 (t % 2) + m and 8 + 4 (t % 2) + m (m = 0..3), as operand
// slots 2m and 2m + 1. Code k of dword d is element 16 (k % 4) + 4 d + k / 4 of the block. Position of
// element K (0..255) of the stretch in that order:
__host__ __device__ inline int perm256_pos(int K) {
    const int g = K >> 6, j = K & 63;
    const int k = 4 * (j & 3) + (j >> 4);   // code index within its dword
    const int d = (j & 15) >> 2;            // dword
    return 32 * (2 * d + ((k >> 2) & 1)) + 8 * g + 2 * (k & 3) + (k >> 3);
}

// C-ABI status codes
enum Status : int {
    kOk = 0,
    kErrShape = -1,       // unsupported shape or argument
    kErrWorkspace = -2,   // workspace / scratch too small
    kErrHip = -3,         // a HIP call failed
    kErrNull = -4,        // required pointer missing
    kErrIo = -5,          // a file could not be read
    kErrSync = -6,        // an earlier persistent call ran out of time waiting for another workgroup
};

// Records the message of the last failure (thread-local) and returns code.
int set_error(int code, const char* fmt, ...);
#define FRT_HIP(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) return ::frt::set_error(::frt::kErrHip, "%s: %s", #call, \
                                                      hipGetErrorString(e_));           \
    } while (0)
#define FRT_LAUNCHED(what)                                                                         \
    do {                                                                                           \
        hipError_t e_ = hipGetLastError();                                                         \
        if (e_ != hipSuccess) return ::frt::set_error(::frt::kErrHip, "%s: %s", what,              \
                                                      hipGetErrorString(e_));                      \
    } while (0)

// Per-kernel timing (off by default): between launches the library records a hipEvent on the
// launch stream; frt_timing_end() turns consecutive events into per-kernel durations. Not for use
// under graph capture.
void timing_mark(hipStream_t stream, const char* kernel);
// Kernels launched through launch_timed() also get start/stop events recorded at the kernel itself
// (hipExtLaunchKernelGGL) while timing is on; frt_timing_end() reports those for the kernel's name,
// which excludes the dispatch gap that an interval between two recorded events also contains.
bool timing_events(const char* kernel, hipEvent_t* start, hipEvent_t* stop);
template <typename K, typename... Args>
inline void launch_timed(const char* name, K kernel, dim3 grid, dim3 block, size_t shm, hipStream_t stream,
                         Args... args) {
    hipEvent_t s, e;
    if (timing_events(name, &s, &e))
        hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(shm), stream, s, e, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, uint32_t(shm), stream, args...);
}

inline size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

// ---- device helpers

// A load through the global address space; p must point into device global memory (an LDS or
// private address given here is read as a global one). Pointers read from memory (the expert blob pointers of
// an entry list) are otherwise generic, and generic (flat) loads share the wait counter of LDS and
// scalar loads, so each LDS or scalar wait after them would also wait for the HBM round trip.
template <class T>
__device__ __forceinline__ T gld(const void* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gld_u4(const void* p) {
    const u32x4_t v = gld<u32x4_t>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// the same as a non-temporal (streaming) load, for expert weights read once per token (measured on
// the decode stack: 0.5% faster than cached loads, same box, alternating runs)
__device__ __forceinline__ uint4 gld_u4_nt(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h2f(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

// fp32 -> fp16 bits, round to nearest even with subnormals, overflow to inf, NaN kept quiet
// (core/fp16.hpp:32-50 semantics), in integer operations: the compiler cannot fuse the rounding
// with the multiply that produced the float (as it does with v_fma_mix for a float conversion).
__host__ __device__ inline uint16_t f32_to_f16_bits(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return uint16_t(sign);
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t sh = 126u - e;
        uint32_t h = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return uint16_t(sign | h);
    }
    uint32_t h = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return uint16_t(sign | h);
}

// fp16 round trip of a float (round to nearest even)
__device__ __forceinline__ float f16_round(float x) { return h2f(f32_to_f16_bits(x)); }

// ---- cross-lane steps on DPP (no LDS round trip). After k pairwise steps every block of 2^k
// lanes holds one value, so the mirror permutations pair whole blocks exactly like an xor would.
#define FRT_DPP(v, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, true))
#define FRT_DPP_ROWS(old, v, ctrl, rows)                                                                    \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, (old)), __builtin_bit_cast(int, (v)), \
                                                          (ctrl), (rows), 0xF, false))
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;       // lane i <-> 15-i within 16
constexpr int kDppBcast15 = 0x142;      // lane 15 of row r to row r+1
constexpr int kDppBcast31 = 0x143;      // lane 31 to rows 2 and 3

// Sum over the wave as the adjacent pairwise tree ((v0+v1)+(v2+v3))+... of the 64 lane values
// (the canonical order of the router logits and the RMS norm); every lane gets the total.
__device__ __forceinline__ float wave_sum_tree(float v) {
    v = v + FRT_DPP(v, kDppXor1);
    v = v + FRT_DPP(v, kDppXor2);
    v = v + FRT_DPP(v, kDppHalfMirror);
    v = v + FRT_DPP(v, kDppMirror);
    v = v + FRT_DPP_ROWS(-0.0f, v, kDppBcast15, 0xA);   // rows 1, 3 += rows 0, 2 (x + -0 == x)
    v = v + FRT_DPP_ROWS(-0.0f, v, kDppBcast31, 0xC);   // rows 2, 3 += row 1
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Sum of the lane values within aligned groups of G lanes (G = 2, 4, 8, 16 or 32), the same
// pairwise tree; the group total is in the group's last lane (and, for G <= 16, in every lane).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    v = v + FRT_DPP(v, kDppXor1);
    if (G >= 4) v = v + FRT_DPP(v, kDppXor2);
    if (G >= 8) v = v + FRT_DPP(v, kDppHalfMirror);
    if (G >= 16) v = v + FRT_DPP(v, kDppMirror);
    if (G >= 32) v = v + FRT_DPP_ROWS(-0.0f, v, kDppBcast15, 0xA);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, FRT_DPP(v, kDppXor1));
    v = fmaxf(v, FRT_DPP(v, kDppXor2));
    v = fmaxf(v, FRT_DPP(v, kDppHalfMirror));
    v = fmaxf(v, FRT_DPP(v, kDppMirror));
    v = fmaxf(v, FRT_DPP_ROWS(-INFINITY, v, kDppBcast15, 0xA));
    v = fmaxf(v, FRT_DPP_ROWS(-INFINITY, v, kDppBcast31, 0xC));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// max within aligned groups of 32 lanes (lanes 0-31 and 32-63), in every lane of the group
__device__ __forceinline__ float half_max(float v) {
    v = fmaxf(v, FRT_DPP(v, kDppXor1));
    v = fmaxf(v, FRT_DPP(v, kDppXor2));
    v = fmaxf(v, FRT_DPP(v, kDppHalfMirror));
    v = fmaxf(v, FRT_DPP(v, kDppMirror));
    v = fmaxf(v, FRT_DPP_ROWS(-INFINITY, v, kDppBcast15, 0xA));   // rows 1, 3 hold the half maxima
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    return (threadIdx.x & 32) ? b : a;
}
__device__ __forceinline__ int wave_sum_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Q8_0 of one 32-value block, as quantize_q8_block (quant/q2_0/q2_0.cpp:93-108):
// d = amax/127 (stored fp16-rounded), id = 1/d from the unrounded d, q = roundf(x * id).
// Division and the products are single correctly rounded IEEE operations (hipcc's default
// correctly rounded fp32 divide), so the codes equal the CPU's bit for bit.
__device__ __forceinline__ int q8_code(float x, float id) { return int(roundf(x * id)); }
__device__ __forceinline__ float q8_scale(float amax) { return amax / 127.0f; }
__device__ __forceinline__ float q8_inv(float d) { return d != 0.0f ? 1.0f / d : 0.0f; }

// 4 x int8 dot with int32 accumulate (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

}  // namespace frt
