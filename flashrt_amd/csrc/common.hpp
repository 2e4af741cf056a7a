// Shared definitions of the MI355X (gfx950) MoE library: the planar Q2_0 layout, error
// plumbing for the C ABI, and small wave64 helpers.
//
// Planar Q2_0 (the reference's repacked layout, quant/q2_0/q2_0.hpp:5-15): a rows x cols matrix
// is codes [rows][cols/64][16] followed by fp16 scales [rows][cols/64]; element j of a 64-block is
// in code byte j % 16 at bits 2*(j/16) and decodes to (q - 1) * d. An expert blob is
// gate [ff][n] | up [ff][n] | down [n][ff].
#pragma once

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

// C-ABI status codes
enum Status : int {
    kOk = 0,
    kErrShape = -1,       // unsupported shape or argument
    kErrWorkspace = -2,   // workspace / scratch too small
    kErrHip = -3,         // a HIP call failed
    kErrNull = -4,        // required pointer missing
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

inline size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

// ---- device helpers

__device__ inline float h2f(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

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
__device__ inline float f16_round(float x) { return h2f(f32_to_f16_bits(x)); }

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ inline int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Q8_0 of one 32-value block, as quantize_q8_block (quant/q2_0/q2_0.cpp:93-108):
// d = amax/127 (stored fp16-rounded), id = 1/d from the unrounded d, q = roundf(x * id).
// Division and the products are single correctly rounded IEEE operations (hipcc's default
// correctly rounded fp32 divide), so the codes equal the CPU's bit for bit.
__device__ inline int q8_code(float x, float id) { return int(roundf(x * id)); }
__device__ inline float q8_scale(float amax) { return amax / 127.0f; }
__device__ inline float q8_inv(float d) { return d != 0.0f ? 1.0f / d : 0.0f; }

// 4 x int8 dot with int32 accumulate (v_dot4_i32_i8)
__device__ inline int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

}  // namespace frt
