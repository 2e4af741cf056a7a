// Seeded synthetic inputs made on the device, so a 48-layer arena (21.7 GB at hidden 2048,
// ff 512) is written in milliseconds instead of being generated on the host and copied.
//
// Recipe (this build's own; the test suite checks it byte for byte against an independent CPU
// restatement):
//   key(seed, cfg, layer, tensor) = mix(mix(mix(mix(seed) ^ cfg) ^ layer) ^ tensor)
//   u64(key, i) = fin(key + (i + 1) * 0x9E3779B97F4A7C15)      SplitMix64 at position i
//   normal(key, i) = sqrt(-2 ln u1) cos(2 pi u2) with u1 = ((r >> 40) + 1) 2^-24,
//                    u2 = ((r >> 16) & 0xFFFFFF) 2^-24, r = u64(key, i); ln and cos as below,
//                    built from +, -, *, /, sqrt only (compiled without contraction), so every
//                    IEEE machine gets the same float (sqrtf and / are the correctly rounded
//                    lowerings; __fsqrt_rn is not, on gfx950).
//   expert blob: matrix m's code byte c = byte c % 8 of u64(key(.., tensor*8 + m), c / 8);
//                scale s = fp16(|normal(key(.., tensor*8 + 3 + m), s)| * sd).
#include "common.hpp"

#include <cmath>
#include <numeric>
#include <vector>

namespace frt {
namespace {

__host__ __device__ inline uint64_t fin(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t mix(uint64_t z) { return fin(z + 0x9E3779B97F4A7C15ull); }
__host__ __device__ inline uint64_t gen_key(uint64_t seed, uint64_t cfg, uint64_t layer, uint64_t tensor) {
    return mix(mix(mix(mix(seed) ^ cfg) ^ layer) ^ tensor);
}
__host__ __device__ inline uint64_t gen_u64(uint64_t key, uint64_t i) { return fin(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

__device__ float det_log(float u) {
    const uint32_t b = __builtin_bit_cast(uint32_t, u);
    const int e = int((b >> 23) & 255) - 127;
    const float m = __builtin_bit_cast(float, (b & 0x7fffffu) | 0x3f800000u);
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 1.0f / 15.0f;
    p = p * s2 + 1.0f / 13.0f;
    p = p * s2 + 1.0f / 11.0f;
    p = p * s2 + 1.0f / 9.0f;
    p = p * s2 + 1.0f / 7.0f;
    p = p * s2 + 1.0f / 5.0f;
    p = p * s2 + 1.0f / 3.0f;
    p = p * s2 + 1.0f;
    const float lnm = 2.0f * s * p;
    return float(e) * 0.693147180559945309f + lnm;
}

__device__ float det_cos2pi(float u) {
    const float x = 6.28318530717958648f * (u - 0.5f);
    const float x2 = x * x;
    float p = 1.0f / 2432902008176640000.0f;
    p = p * x2 - 1.0f / 6402373705728000.0f;
    p = p * x2 + 1.0f / 20922789888000.0f;
    p = p * x2 - 1.0f / 87178291200.0f;
    p = p * x2 + 1.0f / 479001600.0f;
    p = p * x2 - 1.0f / 3628800.0f;
    p = p * x2 + 1.0f / 40320.0f;
    p = p * x2 - 1.0f / 720.0f;
    p = p * x2 + 1.0f / 24.0f;
    p = p * x2 - 0.5f;
    p = p * x2 + 1.0f;
    return -p;
}

__device__ float gen_normal(uint64_t key, uint64_t i) {
    const uint64_t r = gen_u64(key, i);
    const float u1 = float(uint32_t(r >> 40) + 1u) * (1.0f / 16777216.0f);
    const float u2 = float(uint32_t((r >> 16) & 0xFFFFFFull)) * (1.0f / 16777216.0f);
    const float l = det_log(u1);
    return sqrtf(-2.0f * l) * det_cos2pi(u2);
}

// fp16 with round to nearest even of the already rounded float product (integer conversion)
__device__ inline uint16_t to_f16_bits(float v) { return f32_to_f16_bits(v); }

// blockIdx.y = expert index within [e0, e0 + gridDim.y); grid-stride over 8-byte code words and
// scales of one blob. Routed expert e has tensor id e; tensor_base overrides it (shared expert).
__global__ void k_gen_experts(uint64_t seed, int cfg, int layer, int e0, int tensor_base, int n, int ff, float sd,
                              uint8_t* dst, size_t stride) {
    const int e = e0 + blockIdx.y;
    const uint64_t tensor = tensor_base >= 0 ? uint64_t(tensor_base) : uint64_t(e);
    uint8_t* blob = dst + size_t(blockIdx.y) * stride;
    const int rows[3] = {ff, ff, n}, cols[3] = {n, n, ff};
    size_t off = 0;
    for (int m = 0; m < 3; ++m) {
        const size_t nblk = size_t(rows[m]) * (cols[m] / kBlock);
        const uint64_t kc = gen_key(seed, uint64_t(cfg), uint64_t(layer), tensor * 8 + m);
        const uint64_t ks = gen_key(seed, uint64_t(cfg), uint64_t(layer), tensor * 8 + 3 + m);
        uint64_t* codes = reinterpret_cast<uint64_t*>(blob + off);
        const size_t nw = nblk * 2;
        for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < nw; i += size_t(gridDim.x) * blockDim.x)
            codes[i] = gen_u64(kc, i);
        uint16_t* scales = reinterpret_cast<uint16_t*>(blob + off + nblk * 16);
        for (size_t s = blockIdx.x * size_t(blockDim.x) + threadIdx.x; s < nblk; s += size_t(gridDim.x) * blockDim.x)
            scales[s] = to_f16_bits(fabsf(gen_normal(ks, s)) * sd);
        off += nblk * 18;
    }
}

__global__ void k_gen_normal(uint64_t key, float sd, float* dst, size_t count, int round_bf16) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x) {
        float v = gen_normal(key, i) * sd;
        if (round_bf16) {   // round to nearest even bf16, then widen exactly
            uint32_t b = __builtin_bit_cast(uint32_t, v);
            b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
            v = __builtin_bit_cast(float, b);
        }
        dst[i] = v;
    }
}

// x_t = sqrt(rho) * z0 + sqrt(1 - rho) * z_t for t < T (z0 = normal(key0), z_t = normal(key_t)):
// tokens with pairwise correlation rho (a speculative-verify window).
__global__ void k_gen_correlated(uint64_t key0, uint64_t key_base_seed, int cfg, int layer, int tensor0, int T, int n,
                                 float rho, float* dst) {
    const int t = blockIdx.y;
    const uint64_t kt = gen_key(key_base_seed, uint64_t(cfg), uint64_t(layer), uint64_t(tensor0 + 1 + t));
    const float a = sqrtf(rho), b = sqrtf(1.0f - rho);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float p = a * gen_normal(key0, i);
        const float q = b * gen_normal(kt, i);
        dst[size_t(t) * n + i] = p + q;
    }
}

}  // namespace

int gen_experts(uint64_t seed, int cfg, int layer, int e0, int count, int tensor_base, int n, int ff, float sd,
                uint8_t* dst, size_t stride, hipStream_t stream) {
    if (count < 1 || n % kBlock || ff % kBlock || stride < expert_bytes(n, ff))
        return set_error(kErrShape, "gen_experts: bad shape");
    for (int c0 = 0; c0 < count; c0 += 65535) {
        const int c = count - c0 < 65535 ? count - c0 : 65535;
        k_gen_experts<<<dim3(64, c), 256, 0, stream>>>(seed, cfg, layer, e0 + c0, tensor_base, n, ff, sd,
                                                       dst + size_t(c0) * stride, stride);
    }
    FRT_LAUNCHED("gen_experts");
    return kOk;
}

int gen_normal(uint64_t seed, int cfg, int layer, int tensor, float sd, float* dst, size_t count, int round_bf16,
               hipStream_t stream) {
    const uint64_t key = gen_key(seed, uint64_t(cfg), uint64_t(layer), uint64_t(tensor));
    const size_t blocks = (count + 255) / 256 < 4096 ? (count + 255) / 256 : 4096;
    k_gen_normal<<<unsigned(blocks ? blocks : 1), 256, 0, stream>>>(key, sd, dst, count, round_bf16);
    FRT_LAUNCHED("gen_normal");
    return kOk;
}

int gen_correlated(uint64_t seed, int cfg, int layer, int tensor0, int T, int n, float rho, float* dst,
                   hipStream_t stream) {
    const uint64_t key0 = gen_key(seed, uint64_t(cfg), uint64_t(layer), uint64_t(tensor0));
    k_gen_correlated<<<dim3((n + 255) / 256, T), 256, 0, stream>>>(key0, seed, cfg, layer, tensor0, T, n, rho, dst);
    FRT_LAUNCHED("gen_correlated");
    return kOk;
}

// Host: bias[e] = float(-(double)s * alpha * log(1 + perm[e])), perm a Fisher-Yates shuffle of the
// identity with j = u64(key(seed, cfg, layer, 900001), i) % (i + 1), i = E-1 .. 1.
void gen_zipf_bias(uint64_t seed, int cfg, int layer, int E, float s, float alpha, float* bias) {
    std::vector<int> perm(E);
    std::iota(perm.begin(), perm.end(), 0);
    const uint64_t k = gen_key(seed, uint64_t(cfg), uint64_t(layer), 900001ull);
    for (int i = E - 1; i >= 1; --i) {
        const int j = int(gen_u64(k, uint64_t(i)) % uint64_t(i + 1));
        const int t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
    }
    for (int e = 0; e < E; ++e) bias[e] = float(-double(s) * double(alpha) * std::log(1.0 + double(perm[e])));
}

// ---- router / gate tensors of a GGUF file widened to fp32 (exact for every type taken)
namespace {
__global__ void k_widen_f16(const uint16_t* __restrict__ s, size_t n, float* __restrict__ d) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        d[i] = h2f(s[i]);
}
__global__ void k_widen_bf16(const uint16_t* __restrict__ s, size_t n, float* __restrict__ d) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        d[i] = __uint_as_float(uint32_t(s[i]) << 16);
}
// ggml block_q8_0: {fp16 d; int8 qs[32]} (34 bytes); value j of block b = d * qs[j] (exact in fp32)
__global__ void k_widen_q8_0(const uint8_t* __restrict__ s, size_t n, float* __restrict__ d) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const uint8_t* blk = s + (i / 32) * 34;
        const uint16_t dh = uint16_t(blk[0]) | (uint16_t(blk[1]) << 8);
        d[i] = h2f(dh) * float(int8_t(blk[2 + i % 32]));
    }
}
}  // namespace

int router_widen(const void* src, int type, size_t count, float* dst, hipStream_t stream) {
    if (!src || !dst) return set_error(kErrNull, "router_widen: null pointer");
    if (count == 0) return kOk;
    const int grid = int(std::min<size_t>((count + 255) / 256, 4096));
    switch (type) {
        case 0: FRT_HIP(hipMemcpyAsync(dst, src, count * 4, hipMemcpyDeviceToDevice, stream)); return kOk;
        case 1: k_widen_f16<<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(src), count, dst); break;
        case 30: k_widen_bf16<<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(src), count, dst); break;
        case 8:
            if (count % 32) return set_error(kErrShape, "router_widen: Q8_0 count %zu not a multiple of 32", count);
            k_widen_q8_0<<<grid, 256, 0, stream>>>(static_cast<const uint8_t*>(src), count, dst);
            break;
        default: return set_error(kErrShape, "router_widen: ggml type %d (F32, F16, BF16 or Q8_0)", type);
    }
    FRT_LAUNCHED("router_widen");
    return kOk;
}

}  // namespace frt
