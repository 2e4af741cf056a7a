// CPU ORACLE — test infrastructure only (see oracle.h).
//
// The synthetic-input recipe, restated on the CPU so that tests can check the HIP library's
// device-side generator byte for byte. The recipe (this build's own; the reference's tests use
// std::mt19937 and libstdc++'s implementation-defined normal_distribution):
//   key(seed, cfg, layer, tensor) = mix(mix(mix(mix(seed) ^ cfg) ^ layer) ^ tensor)
//   u64(key, i)  = mix(key + (i + 1) * 0x9E3779B97F4A7C15)          (SplitMix64 at position i)
//   mix(z)       = SplitMix64's finaliser: z = (z ^ z>>30) * 0xBF58476D1CE4E5B9;
//                  z = (z ^ z>>27) * 0x94D049BB133111EB; z ^ z>>31
//   normal(key,i): r = u64(key, i); u1 = ((r >> 40) + 1) * 2^-24 in (0, 1];
//                  u2 = ((r >> 16) & 0xFFFFFF) * 2^-24 in [0, 1);
//                  z = sqrt(-2 ln u1) * cos(2 pi u2), in float with the ln and cos below
//                  (only +, -, *, / and sqrt, all correctly rounded, so any IEEE machine agrees).
// Expert blob (planar Q2_0, gate | up | down): matrix m's code byte c = byte (c % 8) of
// u64(key(seed,cfg,layer,tensor*8 + m), c / 8); scale s = fp16(|normal(key(..., tensor*8+3+m), s)| * sd).
// Routed expert e has tensor = e; the shared expert tensor = 100000.
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <numeric>
#include <vector>

namespace {

inline uint64_t fin(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
inline uint64_t mix(uint64_t z) { return fin(z + 0x9E3779B97F4A7C15ull); }

// ln(u), u in (0, 1]: u = m * 2^e, m in [1, 2); ln m = 2 atanh(s), s = (m-1)/(m+1) in [0, 1/3)
float det_log(float u) {
    uint32_t b;
    std::memcpy(&b, &u, 4);
    const int e = int((b >> 23) & 255) - 127;
    const uint32_t mb = (b & 0x7fffffu) | 0x3f800000u;
    float m;
    std::memcpy(&m, &mb, 4);
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

// cos(2 pi u), u in [0, 1): cos(2 pi u) = -cos(x), x = 2 pi (u - 1/2) in [-pi, pi); Taylor to x^20
float det_cos2pi(float u) {
    const float x = 6.28318530717958648f * (u - 0.5f);
    const float x2 = x * x;
    float p = 1.0f / 2432902008176640000.0f;    // 1/20!
    p = p * x2 - 1.0f / 6402373705728000.0f;    // 1/18!
    p = p * x2 + 1.0f / 20922789888000.0f;      // 1/16!
    p = p * x2 - 1.0f / 87178291200.0f;         // 1/14!
    p = p * x2 + 1.0f / 479001600.0f;           // 1/12!
    p = p * x2 - 1.0f / 3628800.0f;             // 1/10!
    p = p * x2 + 1.0f / 40320.0f;               // 1/8!
    p = p * x2 - 1.0f / 720.0f;                 // 1/6!
    p = p * x2 + 1.0f / 24.0f;
    p = p * x2 - 0.5f;
    p = p * x2 + 1.0f;   // cos(x)
    return -p;
}

}  // namespace

extern "C" {

uint64_t orc_gen_key(uint64_t seed, uint64_t cfg, uint64_t layer, uint64_t tensor) {
    return mix(mix(mix(mix(seed) ^ cfg) ^ layer) ^ tensor);
}

uint64_t orc_gen_u64(uint64_t key, uint64_t i) { return fin(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

float orc_gen_normal(uint64_t key, uint64_t i) {
    const uint64_t r = orc_gen_u64(key, i);
    const float u1 = float((r >> 40) + 1) * (1.0f / 16777216.0f);
    const float u2 = float((r >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
    const float l = det_log(u1);
    const float rad = std::sqrt(-2.0f * l);
    return rad * det_cos2pi(u2);
}

void orc_gen_expert(uint64_t seed, int cfg, int layer, int expert, int n, int ff, float scale_sd, uint8_t* blob) {
    const int rows[3] = {ff, ff, n}, cols[3] = {n, n, ff};
    size_t off = 0;
    for (int m = 0; m < 3; ++m) {
        const size_t nblk = size_t(rows[m]) * (cols[m] / 64);
        const uint64_t kc = orc_gen_key(seed, uint64_t(cfg), uint64_t(layer), uint64_t(expert) * 8 + m);
        const uint64_t ks = orc_gen_key(seed, uint64_t(cfg), uint64_t(layer), uint64_t(expert) * 8 + 3 + m);
        uint8_t* codes = blob + off;
        for (size_t c = 0; c < nblk * 16; c += 8) {
            const uint64_t r = orc_gen_u64(kc, c / 8);
            std::memcpy(codes + c, &r, 8);   // little-endian: byte c%8 = bits 8*(c%8)
        }
        auto* scales = reinterpret_cast<uint16_t*>(codes + nblk * 16);
        for (size_t s = 0; s < nblk; ++s) {
            const float v = std::fabs(orc_gen_normal(ks, s)) * scale_sd;
            const uint16_t h = orc_f32_to_f16(v);
            std::memcpy(scales + s, &h, 2);
        }
        off += nblk * 18;
    }
}

void orc_gen_normal_f32(uint64_t seed, int cfg, int layer, int tensor, float sd, float* dst, size_t count) {
    const uint64_t k = orc_gen_key(seed, uint64_t(cfg), uint64_t(layer), uint64_t(tensor));
    for (size_t i = 0; i < count; ++i) dst[i] = orc_gen_normal(k, i) * sd;
}

// Fisher-Yates from the identity with j = u64(key, i) % (i + 1) for i = E-1 .. 1; expert e's rank
// is perm[e]; bias[e] = float(-(double)s * alpha * log(1 + perm[e])).
void orc_gen_zipf_bias(uint64_t seed, int cfg, int layer, int E, float s, float alpha, float* bias) {
    std::vector<int> perm(E);
    std::iota(perm.begin(), perm.end(), 0);
    const uint64_t k = orc_gen_key(seed, uint64_t(cfg), uint64_t(layer), 900001ull);
    for (int i = E - 1; i >= 1; --i) {
        const int j = int(orc_gen_u64(k, uint64_t(i)) % uint64_t(i + 1));
        std::swap(perm[i], perm[j]);
    }
    for (int e = 0; e < E; ++e) bias[e] = float(-double(s) * double(alpha) * std::log(1.0 + double(perm[e])));
}

}  // extern "C"
