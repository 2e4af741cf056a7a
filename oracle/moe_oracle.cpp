// CPU ORACLE — test infrastructure only (see oracle.h). Not part of the product path.
//
// Clean-room restatement of the reference's CPU MoE arithmetic. Compiled with
// -ffp-contract=off: every multiply-add below is either two rounded operations or an explicit
// fmaf, exactly as stated, so the float order is defined by this source alone.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr int kBlock = 64;     // weights per Q2_0 block (quant/q2_0/q2_0.hpp:23)
constexpr int kQ8 = 32;        // activations per Q8_0 block (q2_0.hpp:25)

struct MatV {
    const uint8_t* codes;
    const uint16_t* scales;
    int rows, cols;
    int nb() const { return cols / kBlock; }
};

// codes [rows][cols/64][16], then fp16 scales [rows][cols/64] (q2_0.cpp:48-52)
MatV mat_view(const uint8_t* p, int rows, int cols) {
    const size_t nblk = size_t(rows) * (cols / kBlock);
    return MatV{p, reinterpret_cast<const uint16_t*>(p + nblk * 16), rows, cols};
}

struct ExpertV {
    MatV gate, up, down;
};
// blob = gate [ff][n] | up [ff][n] | down [n][ff] (q2_0.cpp:66-72)
ExpertV expert_view(const uint8_t* blob, int n, int ff) {
    const size_t gu = orc_mat_bytes(ff, n);
    return ExpertV{mat_view(blob, ff, n), mat_view(blob + gu, ff, n), mat_view(blob + 2 * gu, n, ff)};
}

// Quantized activation with the VNNI kernel's helper vectors (q2_0.hpp:58-72).
struct Act {
    const int8_t* qs;
    const float* d;
};

// Σ_{j<32} (code_j - 1) * a_j for half k of block b (integer exact, any order).
inline int half_dot(const uint8_t* blk, const int8_t* a, int k) {
    int s = 0;
    for (int j = 0; j < kQ8; ++j) s += (orc_planar_code(blk, k * kQ8 + j) - 1) * a[k * kQ8 + j];
    return s;
}

// matvec_ref order (q2_0.cpp:119-140): per block sumi = Σ_k d_a * float(s) from 0, then
// sumf += d_w * sumi, blocks ascending.
void matvec_ref(const MatV& w, const Act* a, int ntok, int r0, int r1, float* y, int ldy) {
    const int nb = w.nb();
    for (int t = 0; t < ntok; ++t)
        for (int r = r0; r < r1; ++r) {
            float sumf = 0.0f;
            for (int b = 0; b < nb; ++b) {
                const uint8_t* blk = w.codes + (size_t(r) * nb + b) * 16;
                const float d0 = orc_f16_to_f32(w.scales[size_t(r) * nb + b]);
                float sumi = 0.0f;
                for (int k = 0; k < 2; ++k) {
                    const int s = half_dot(blk, a[t].qs + b * kBlock, k);
                    const float p = a[t].d[2 * b + k] * float(s);
                    sumi = sumi + p;
                }
                const float p = d0 * sumi;
                sumf = sumf + p;
            }
            y[size_t(t) * ldy + r] = sumf;
        }
}

// The AVX-512 VNNI kernel's float order (q2_0_avx512.cpp:23-52): 16 dword lanes; lane L = 4i + w
// covers elements 16i + 4w .. +3 of each block (the planar broadcast + per-lane shift), with
// s = Σ (q-1)a over those 4 elements (vpdpbusd onto negsum4), f = float(s) * d_a(lane half),
// acc_L = fma(f, d_w, acc_L) over blocks ascending; then GCC's _mm512_reduce_add_ps tree:
// halves (L, L+8), then (L, L+4), then (L, L+2), then (0, 1).
void matvec_vnni(const MatV& w, const Act* a, int ntok, int r0, int r1, float* y, int ldy) {
    const int nb = w.nb();
    for (int t = 0; t < ntok; ++t)
        for (int r = r0; r < r1; ++r) {
            float acc[16] = {};
            for (int b = 0; b < nb; ++b) {
                const uint8_t* blk = w.codes + (size_t(r) * nb + b) * 16;
                const float dw = orc_f16_to_f32(w.scales[size_t(r) * nb + b]);
                const int8_t* ab = a[t].qs + b * kBlock;
                for (int L = 0; L < 16; ++L) {
                    int s = 0;
                    for (int c = 0; c < 4; ++c) {
                        const int j = 4 * L + c;   // activation element of this dword lane
                        s += (orc_planar_code(blk, j) - 1) * ab[j];
                    }
                    const float f = float(s) * a[t].d[2 * b + (L >= 8)];
                    acc[L] = std::fmaf(f, dw, acc[L]);
                }
            }
            float h8[8], h4[4], h2[2];
            for (int i = 0; i < 8; ++i) h8[i] = acc[i + 8] + acc[i];
            for (int i = 0; i < 4; ++i) h4[i] = h8[i + 4] + h8[i];
            for (int i = 0; i < 2; ++i) h2[i] = h4[i + 2] + h4[i];
            y[size_t(t) * ldy + r] = h2[1] + h2[0];
        }
}

void matvec(const MatV& w, const Act* a, int ntok, int r0, int r1, float* y, int ldy, int order) {
    if (order == 1) matvec_vnni(w, a, ntok, r0, r1, y, ldy);
    else matvec_ref(w, a, ntok, r0, r1, y, ldy);
}

// silu(g) * u with libm exp, as q2_0.cpp:180 and moe_cpu.cpp:58
inline float swiglu(float g, float u) {
    const float e = std::exp(-g);
    const float den = 1.0f + e;
    const float s = g / den;
    return s * u;
}

// quantize_q8_block (q2_0.cpp:93-108): amax; d = amax/127; id = d != 0 ? 1/d : 0 (unrounded d);
// stored d is fp16-rounded; q = (int8) roundf(x * id)
void quant_block(const float* x32, int8_t* q, float* d) {
    float amax = 0.0f;
    for (int j = 0; j < kQ8; ++j) amax = std::max(amax, std::fabs(x32[j]));
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    *d = orc_f16_to_f32(orc_f32_to_f16(dd));
    for (int j = 0; j < kQ8; ++j) q[j] = int8_t(std::roundf(x32[j] * id));
}

// The canonical reduction of 64 chain sums: the adjacent pairwise tree
// ((s0+s1)+(s2+s3))+... (level by level, pairs of neighbouring blocks).
float tree64(float* s) {
    for (int step = 1; step < 64; step *= 2)
        for (int j = 0; j < 64; j += 2 * step) s[j] = s[j] + s[j + step];
    return s[0];
}

}  // namespace

extern "C" {

// core/fp16.hpp:11-30
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int ex = 113;   // 127 - 15 + 1
            while (!(m & 0x400)) {
                m <<= 1;
                --ex;
            }
            bits = sign | (uint32_t(ex) << 23) | ((m & 0x3ff) << 13);
        }
    } else if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// core/fp16.hpp:32-50: round to nearest even, subnormals, overflow to inf, NaN kept quiet
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000;
    const uint32_t ax = x & 0x7fffffff;
    if (ax >= 0x7f800000) return uint16_t(sign | 0x7c00 | (ax > 0x7f800000 ? 0x200 : 0));
    if (ax >= 0x477ff000) return uint16_t(sign | 0x7c00);
    if (ax < 0x38800000) {
        if (ax < 0x33000000) return uint16_t(sign);
        const uint32_t e = ax >> 23, m = (ax & 0x7fffff) | 0x800000;
        const uint32_t sh = 126 - e;
        uint32_t h = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return uint16_t(sign | h);
    }
    uint32_t h = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
    return uint16_t(sign | h);
}

size_t orc_mat_bytes(int rows, int cols) { return size_t(rows) * (cols / kBlock) * 18; }   // q2_0.cpp:44
size_t orc_expert_bytes(int n, int ff) { return 2 * orc_mat_bytes(ff, n) + orc_mat_bytes(n, ff); }   // q2_0.cpp:64

// planar: element j of a block is in byte j%16 at bits 2*(j/16) (q2_0.hpp:11-13)
int orc_planar_code(const uint8_t* blk16, int j) { return (blk16[j % 16] >> (2 * (j / 16))) & 3; }

// repack (q2_0.cpp:54-62), written as the element-wise placement of tests/test_q2_0.cpp:74-86
void orc_repack(const void* ggml_rows, int rows, int cols, void* dst) {
    const auto* in = static_cast<const uint8_t*>(ggml_rows);
    auto* codes = static_cast<uint8_t*>(dst);
    const size_t nblk = size_t(rows) * (cols / kBlock);
    auto* scales = reinterpret_cast<uint16_t*>(codes + nblk * 16);
    for (size_t i = 0; i < nblk; ++i) {
        const uint8_t* b = in + i * 18;   // {u16 d; u8 qs[16]}
        uint8_t out[16] = {};
        for (int j = 0; j < kBlock; ++j) {
            const int q = (b[2 + j / 4] >> (2 * (j % 4))) & 3;   // ggml: byte j/4, bits 2*(j%4)
            out[j % 16] |= uint8_t(q << (2 * (j / 16)));
        }
        std::memcpy(codes + i * 16, out, 16);
        uint16_t d;
        std::memcpy(&d, b, 2);
        scales[i] = d;
    }
}

void orc_quantize_q8(const float* x, int n, int8_t* qs, float* d) {
    for (int i = 0; i < n / kQ8; ++i) quant_block(x + size_t(i) * kQ8, qs + size_t(i) * kQ8, d + i);
}

// Q8 in blocks of blk = 32 or 64 values: quant_block's rule over blk values (moe_q2's block64
// activations, kernels/cuda/moe_q2.cu:58-81 with AB = 64; d fp16-rounded as the CPU path stores it).
// The scales are stored one per 32 values (a 64-block's repeated), the layout matvec reads, so that
// the per-block product d_w * d_a * sum over 64 is formed as two halves of 32 with the same d_a.
void orc_quantize_q8_blk(const float* x, int n, int blk, int8_t* qs, float* d) {
    if (blk != 64) return orc_quantize_q8(x, n, qs, d);
    for (int i = 0; i < n / 64; ++i) {
        const float* xb = x + size_t(i) * 64;
        float amax = 0.0f;
        for (int j = 0; j < 64; ++j) amax = std::max(amax, std::fabs(xb[j]));
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        d[2 * i] = d[2 * i + 1] = orc_f16_to_f32(orc_f32_to_f16(dd));
        for (int j = 0; j < 64; ++j) qs[size_t(i) * 64 + j] = int8_t(std::roundf(xb[j] * id));
    }
}

void orc_matvec(const uint8_t* w, int rows, int cols, const int8_t* qs, const float* d, int ntok, int r0, int r1,
                float* y, int ldy, int order) {
    const MatV m = mat_view(w, rows, cols);
    std::vector<Act> a(ntok);
    for (int t = 0; t < ntok; ++t) a[t] = Act{qs + size_t(t) * cols, d + size_t(t) * (cols / kQ8)};
    matvec(m, a.data(), ntok, r0, r1, y, ldy, order);
}

// expert_ffn (q2_0.cpp:164-185): gate, up, SwiGLU, Q8 of h, down
void orc_expert_ffn(const uint8_t* blob, int n, int ff, const int8_t* xq, const float* xd, int ntok, float* out, int ldo,
                    int order) {
    orc_expert_ffn_blk(blob, n, ff, xq, xd, ntok, out, ldo, order, kQ8);
}

// expert_ffn with h quantized in blocks of hblk = 32 or 64 (orc_quantize_q8_blk)
void orc_expert_ffn_blk(const uint8_t* blob, int n, int ff, const int8_t* xq, const float* xd, int ntok, float* out,
                        int ldo, int order, int hblk) {
    const ExpertV e = expert_view(blob, n, ff);
    std::vector<Act> a(ntok), ha(ntok);
    for (int t = 0; t < ntok; ++t) a[t] = Act{xq + size_t(t) * n, xd + size_t(t) * (n / kQ8)};
    std::vector<float> g(size_t(ntok) * ff), u(size_t(ntok) * ff);
    std::vector<int8_t> hq(size_t(ntok) * ff);
    std::vector<float> hd(size_t(ntok) * (ff / kQ8));
    matvec(e.gate, a.data(), ntok, 0, ff, g.data(), ff, order);
    matvec(e.up, a.data(), ntok, 0, ff, u.data(), ff, order);
    for (int t = 0; t < ntok; ++t) {
        float* gt = g.data() + size_t(t) * ff;
        const float* ut = u.data() + size_t(t) * ff;
        for (int i = 0; i < ff; ++i) gt[i] = swiglu(gt[i], ut[i]);
        orc_quantize_q8_blk(gt, ff, hblk, hq.data() + size_t(t) * ff, hd.data() + size_t(t) * (ff / kQ8));
        ha[t] = Act{hq.data() + size_t(t) * ff, hd.data() + size_t(t) * (ff / kQ8)};
    }
    matvec(e.down, ha.data(), ntok, 0, n, out, ldo, order);
}

float orc_dot_canon(const float* w, const float* x, int n) {
    const int L = n / 64;
    float s[64];
    for (int j = 0; j < 64; ++j) {
        float acc = 0.0f;
        for (int k = j * L; k < (j + 1) * L; ++k) acc = std::fmaf(w[k], x[k], acc);
        s[j] = acc;
    }
    return tree64(s);
}

// The RMS norm of the stack's input in this build's canonical order (no reference test pins one; the
// GPU kernels share it, topk.hpp rms_scale_wave): per chain of n / 64 contiguous values, four
// contiguous quarters each summed by fmaf from 0, (q0 + q1) + (q2 + q3), then the pairwise tree.
void orc_rmsnorm(const float* x, int T, int n, float* u) {
    const int L = n / 64;
    for (int t = 0; t < T; ++t) {
        const float* xt = x + size_t(t) * n;
        float s[64];
        for (int j = 0; j < 64; ++j) {   // chain j in four quarters, each an fmaf chain from 0
            float q[4];
            for (int c = 0; c < 4; ++c) {
                q[c] = 0.0f;
                for (int k = j * L + c * (L / 4); k < j * L + (c + 1) * (L / 4); ++k) q[c] = std::fmaf(xt[k], xt[k], q[c]);
            }
            s[j] = (q[0] + q[1]) + (q[2] + q[3]);
        }
        const float ms = tree64(s) / float(n);
        const float r = 1.0f / std::sqrt(ms + 1e-6f);
        for (int i = 0; i < n; ++i) u[size_t(t) * n + i] = xt[i] * r;
    }
}

void orc_router_logits(const float* x, int T, const float* W, const float* bias, int E, int n, float* logits) {
    for (int t = 0; t < T; ++t)
        for (int e = 0; e < E; ++e) {
            float v = orc_dot_canon(W + size_t(e) * n, x + size_t(t) * n, n);
            if (bias) v = v + bias[e];
            logits[size_t(t) * E + e] = v;
        }
}

// moe_ref.cu:146-164: mx = max; p_e = exp(l_e - mx) in float, summed in double; p = float(p/sum);
// top-K; wsum = float sum of the selected p in rank order, clamped at 6.103515625e-5; w = p/wsum.
// Rank: logit descending, ties to the lower id (test_route_topk.cpp:52-55).
void orc_route_topk(const float* logits, int T, int E, int K, int32_t* ids, float* wts, uint32_t* counts) {
    std::vector<float> p(E);
    std::vector<int> idx(E);
    for (int t = 0; t < T; ++t) {
        const float* lg = logits + size_t(t) * E;
        const float mx = *std::max_element(lg, lg + E);
        double sum = 0;
        for (int e = 0; e < E; ++e) {
            p[e] = std::exp(lg[e] - mx);
            sum += p[e];
        }
        for (int e = 0; e < E; ++e) p[e] = float(double(p[e]) / sum);
        for (int e = 0; e < E; ++e) idx[e] = e;
        std::partial_sort(idx.begin(), idx.begin() + K, idx.end(),
                          [&](int a, int b) { return lg[a] > lg[b] || (lg[a] == lg[b] && a < b); });
        float wsum = 0.0f;
        for (int k = 0; k < K; ++k) wsum += p[idx[k]];
        wsum = std::max(wsum, 6.103515625e-5f);
        for (int k = 0; k < K; ++k) {
            ids[size_t(t) * K + k] = idx[k];
            wts[size_t(t) * K + k] = p[idx[k]] / wsum;
            if (counts) ++counts[idx[k]];
        }
    }
}

void orc_dispatch(const int32_t* ids, int T, int K, int E, int32_t* bounds, int32_t* tok_of, int32_t* slot_of) {
    std::vector<int32_t> cnt(E + 1, 0);
    const int S = T * K;
    for (int s = 0; s < S; ++s) ++cnt[ids[s] + 1];
    for (int e = 0; e < E; ++e) cnt[e + 1] += cnt[e];
    for (int e = 0; e <= E; ++e) bounds[e] = cnt[e];
    for (int s = 0; s < S; ++s) {
        const int r = cnt[ids[s]]++;
        slot_of[r] = s;
        tok_of[r] = s / K;
    }
}

// moe_cpu (quant/q2_0/moe_cpu.cpp:36-114). Phase A items (miss, 32-row chunk): gate/up rows,
// SwiGLU, Q8 of that block of h. Phase B items (64 output rows): out rows zeroed for every token
// of the window, then out[tok] += w * down(h) for each miss in list order.
void orc_moe_cpu(int n, int ff, const uint8_t* const* blobs, const int* ntok, const int* tok, const float* w, int n_miss,
                 const int8_t* xq, const float* xd, int T, float* out, int ldo, int n_threads, int order) {
    std::vector<int8_t> hq(size_t(n_miss) * 4 * ff);
    std::vector<float> hd(size_t(n_miss) * 4 * (ff / kQ8));
    std::atomic<int> next_a{0}, next_b{0};
    const int na = ff / kQ8, nbk = n / 64;
    auto phase_a = [&]() {
        std::vector<float> g(size_t(4) * ff), u(size_t(4) * ff);
        for (int k; (k = next_a.fetch_add(1)) < n_miss * na;) {
            const int i = k / na, r0 = (k % na) * kQ8;
            const ExpertV e = expert_view(blobs[i], n, ff);
            Act xa[4];
            for (int j = 0; j < ntok[i]; ++j) {
                const int t = tok[i * 4 + j];
                xa[j] = Act{xq + size_t(t) * n, xd + size_t(t) * (n / kQ8)};
            }
            matvec(e.gate, xa, ntok[i], r0, r0 + kQ8, g.data(), ff, order);
            matvec(e.up, xa, ntok[i], r0, r0 + kQ8, u.data(), ff, order);
            for (int j = 0; j < ntok[i]; ++j) {
                float h32[kQ8];
                for (int r = 0; r < kQ8; ++r) h32[r] = swiglu(g[size_t(j) * ff + r0 + r], u[size_t(j) * ff + r0 + r]);
                quant_block(h32, hq.data() + (size_t(i) * 4 + j) * ff + r0,
                            hd.data() + (size_t(i) * 4 + j) * (ff / kQ8) + r0 / kQ8);
            }
        }
    };
    auto phase_b = [&]() {
        std::vector<float> tv(size_t(4) * n);
        for (int k; (k = next_b.fetch_add(1)) < nbk;) {
            const int r0 = k * 64;
            for (int t = 0; t < T; ++t) std::memset(out + size_t(t) * ldo + r0, 0, 64 * 4);
            for (int i = 0; i < n_miss; ++i) {
                const ExpertV e = expert_view(blobs[i], n, ff);
                Act ha[4];
                for (int j = 0; j < ntok[i]; ++j)
                    ha[j] = Act{hq.data() + (size_t(i) * 4 + j) * ff, hd.data() + (size_t(i) * 4 + j) * (ff / kQ8)};
                matvec(e.down, ha, ntok[i], r0, r0 + 64, tv.data(), n, order);
                for (int j = 0; j < ntok[i]; ++j) {
                    float* o = out + size_t(tok[i * 4 + j]) * ldo;
                    const float wj = w[i * 4 + j];
                    for (int r = r0; r < r0 + 64; ++r) {
                        const float p = wj * tv[size_t(j) * n + r];
                        o[r] = o[r] + p;
                    }
                }
            }
        }
    };
    if (n_threads <= 1) {
        phase_a();
        phase_b();
        return;
    }
    std::vector<std::thread> th;
    for (int i = 0; i < n_threads; ++i) th.emplace_back(phase_a);
    for (auto& x : th) x.join();
    th.clear();
    for (int i = 0; i < n_threads; ++i) th.emplace_back(phase_b);
    for (auto& x : th) x.join();
}

void orc_moe_layer(const uint8_t* arena, size_t stride, int E, const uint8_t* shared_blob, const float* router_w,
                   const float* router_bias, const float* gate_w, int n, int ff, int K, const float* x, int T,
                   int n_threads, int order, float* out, int32_t* ids, float* wts, float* logits_out, int norm_input) {
    orc_moe_layer_shexp(arena, stride, E, -1, nullptr, nullptr, nullptr, 0, shared_blob, router_w, router_bias, gate_w, n,
                        ff, K, x, T, n_threads, order, out, ids, wts, logits_out, norm_input);
}

namespace {
// one weight of row r, column j of a dense [rows][cols] matrix of ggml type F32 / F16 / BF16
float dense_w(int type, const void* w, int cols, int r, int j) {
    const size_t i = size_t(r) * cols + j;
    if (type == 0) return static_cast<const float*>(w)[i];
    const uint16_t b = static_cast<const uint16_t*>(w)[i];
    if (type == 1) return orc_f16_to_f32(b);
    uint32_t u = uint32_t(b) << 16;   // bf16: the upper half of an fp32
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
// y[r] = row r of W (rows x cols) . a, for one activation vector
void dense_mv(int type, const void* w, int rows, int cols, const float* a, const int8_t* aq, const float* ad,
              float* y) {
    for (int r = 0; r < rows; ++r) {
        if (type == 8) {   // Q8_0: 34-byte blocks {fp16 d; int8 q[32]}, ggml_vec_dot_q8_0_q8_0
            const uint8_t* row = static_cast<const uint8_t*>(w) + size_t(r) * (cols / kQ8) * 34;
            float sumf = 0.0f;
            for (int b = 0; b < cols / kQ8; ++b) {
                const uint8_t* blk = row + size_t(b) * 34;
                uint16_t db;
                std::memcpy(&db, blk, 2);
                const int8_t* q = reinterpret_cast<const int8_t*>(blk + 2);
                int sumi = 0;
                for (int j = 0; j < kQ8; ++j) sumi += int(q[j]) * int(aq[b * kQ8 + j]);
                const float dd = orc_f16_to_f32(db) * ad[b];
                sumf += float(sumi) * dd;
            }
            y[r] = sumf;
        } else {
            double s = 0.0;
            for (int j = 0; j < cols; ++j) s += double(dense_w(type, w, cols, r, j) * a[j]);
            y[r] = float(s);
        }
    }
}
}  // namespace

void orc_dense_mv(int type, const void* w, int rows, int cols, const float* x, int T, float* y) {
    std::vector<int8_t> xq(cols);
    std::vector<float> xd(cols / kQ8);
    for (int t = 0; t < T; ++t) {
        const float* xt = x + size_t(t) * cols;
        if (type == 8) orc_quantize_q8(xt, cols, xq.data(), xd.data());
        dense_mv(type, w, rows, cols, xt, xq.data(), xd.data(), y + size_t(t) * rows);
    }
}

void orc_shexp_ffn(int type, const void* gate, const void* up, const void* down, int n, int ffs, const float* x, int T,
                   float* out) {
    std::vector<float> g(ffs), u(ffs);
    std::vector<int8_t> xq(n), hq(ffs);
    std::vector<float> xd(n / kQ8), hd(ffs / kQ8);
    for (int t = 0; t < T; ++t) {
        const float* xt = x + size_t(t) * n;
        if (type == 8) orc_quantize_q8(xt, n, xq.data(), xd.data());
        dense_mv(type, gate, ffs, n, xt, xq.data(), xd.data(), g.data());
        dense_mv(type, up, ffs, n, xt, xq.data(), xd.data(), u.data());
        for (int i = 0; i < ffs; ++i) g[i] = swiglu(g[i], u[i]);
        if (type == 8) orc_quantize_q8(g.data(), ffs, hq.data(), hd.data());
        dense_mv(type, down, n, ffs, g.data(), hq.data(), hd.data(), out + size_t(t) * n);
    }
}

void orc_moe_layer_shexp(const uint8_t* arena, size_t stride, int E, int shared_type, const void* sg, const void* su,
                         const void* sd, int ffs, const uint8_t* shared_blob, const float* router_w,
                         const float* router_bias, const float* gate_w, int n, int ff, int K, const float* x, int T,
                         int n_threads, int order, float* out, int32_t* ids, float* wts, float* logits_out,
                         int norm_input) {
    std::vector<float> un;
    if (norm_input) {
        un.resize(size_t(T) * n);
        orc_rmsnorm(x, T, n, un.data());
        x = un.data();
    }
    std::vector<float> logits(size_t(T) * E);
    orc_router_logits(x, T, router_w, router_bias, E, n, logits.data());
    if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);
    orc_route_topk(logits.data(), T, E, K, ids, wts, nullptr);
    std::vector<int8_t> xq(size_t(T) * n);
    std::vector<float> xd(size_t(T) * (n / kQ8));
    orc_quantize_q8(x, T * n, xq.data(), xd.data());
    // per expert, the tokens routed to it in token order (moe_ref.cu:145, 166), <= 4 per miss
    std::vector<std::vector<std::pair<int, float>>> routed(E);
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < K; ++k) routed[ids[size_t(t) * K + k]].push_back({t, wts[size_t(t) * K + k]});
    std::vector<const uint8_t*> blobs;
    std::vector<int> nt, tk;
    std::vector<float> wv;
    for (int e = 0; e < E; ++e)
        for (size_t i = 0; i < routed[e].size(); i += 4) {
            blobs.push_back(arena + size_t(e) * stride);
            int c = 0;
            for (size_t j = i; j < std::min(routed[e].size(), i + 4); ++j, ++c) {
                tk.push_back(routed[e][j].first);
                wv.push_back(routed[e][j].second);
            }
            nt.push_back(c);
            for (; c < 4; ++c) {
                tk.push_back(0);
                wv.push_back(0.0f);
            }
        }
    std::vector<float> moe(size_t(T) * n);
    orc_moe_cpu(n, ff, blobs.data(), nt.data(), tk.data(), wv.data(), int(blobs.size()), xq.data(), xd.data(), T,
                moe.data(), n, n_threads, order);
    // the shared expert and its sigmoid gate, added as k_add_gated (moe_ref.cu:90-97)
    for (int t0 = 0; t0 < T; t0 += 4) {
        const int c = std::min(4, T - t0);
        std::vector<float> shc(size_t(c) * n);
        if (shared_type >= 0)
            orc_shexp_ffn(shared_type, sg, su, sd, n, ffs, x + size_t(t0) * n, c, shc.data());
        else
            orc_expert_ffn(shared_blob, n, ff, xq.data() + size_t(t0) * n, xd.data() + size_t(t0) * (n / kQ8), c,
                           shc.data(), n, order);
        for (int t = t0; t < t0 + c; ++t) {
            const float gl = orc_dot_canon(gate_w, x + size_t(t) * n, n);
            const float g = 1.0f / (1.0f + std::exp(-gl));
            for (int i = 0; i < n; ++i) {
                const float p = shc[size_t(t - t0) * n + i] * g;
                out[size_t(t) * n + i] = moe[size_t(t) * n + i] + p;
            }
        }
    }
}

}  // extern "C"
