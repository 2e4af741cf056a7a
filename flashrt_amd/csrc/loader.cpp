// Q2_0 repack (ggml block order -> planar) and the expert loader into the HBM arena.
//
// Repack (quant/q2_0/q2_0.cpp:21-62 repack, :64-80 repack_expert): a ggml block {fp16 d; u8 qs[16]}
// holds element j of 64 at byte j / 4, bits 2 (j % 4); the planar layout holds it at byte j % 16,
// bits 2 (j / 16), codes of a matrix first ([rows][cols/64][16]), then its fp16 scales
// ([rows][cols/64]). Written as words: planar bytes 4w .. 4w + 3 are elements 4w + b + 16p
// (b = 0..3, p = 0..3), which are field b of ggml byte w + 4p, so planar word w is the OR over p of
// spread(qs[w + 4p]) << 2p, where spread() moves the four 2-bit fields of a byte to bits 0-1 of
// four bytes.
//
// Loader (arch/qwen4exp/experts.cpp:65-131 load_experts): work items of 32 experts of one layer;
// each worker thread reads the item's three slab ranges with O_DIRECT (buffered where the file
// system refuses O_DIRECT), repacks each expert into a pinned staging buffer laid out at the
// arena's stride, and uploads the item with one copy to its place in the HBM arena.
#include "common.hpp"

#include "../../include/flashrt_moe.h"

#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace frt {

namespace {

inline uint32_t spread2(uint32_t x) {
    return (x & 3u) | ((x & 0x0Cu) << 6) | ((x & 0x30u) << 12) | ((x & 0xC0u) << 18);
}

// one 64-element block: 16 ggml code bytes -> 16 planar code bytes
inline void repack_codes(const uint8_t* qs, uint8_t* out) {
    for (int w = 0; w < 4; ++w) {
        const uint32_t v = spread2(qs[w]) | (spread2(qs[w + 4]) << 2) | (spread2(qs[w + 8]) << 4) | (spread2(qs[w + 12]) << 6);
        out[4 * w] = uint8_t(v);
        out[4 * w + 1] = uint8_t(v >> 8);
        out[4 * w + 2] = uint8_t(v >> 16);
        out[4 * w + 3] = uint8_t(v >> 24);
    }
}

constexpr size_t kGgmlBlock = 18;   // fp16 scale, then 16 code bytes

size_t repack_mat(const uint8_t* in, int rows, int cols, uint8_t* dst) {
    const size_t nblk = size_t(rows) * (cols / kBlock);
    uint8_t* scales = dst + nblk * 16;
    for (size_t i = 0; i < nblk; ++i) {
        const uint8_t* b = in + i * kGgmlBlock;
        repack_codes(b + 2, dst + i * 16);
        scales[2 * i] = b[0];
        scales[2 * i + 1] = b[1];
    }
    return nblk * kGgmlBlock;
}

struct FdCloser {
    int fd = -1;
    ~FdCloser() {
        if (fd >= 0) close(fd);
    }
};

constexpr size_t kAlign = 4096;
constexpr int kExpertsPerItem = 32;

}  // namespace

}  // namespace frt

using namespace frt;

extern "C" {

size_t frt_q2_repack(const void* ggml_rows, int rows, int cols, void* dst) {
    if (!ggml_rows || !dst || rows < 1 || cols < kBlock || cols % kBlock) {
        set_error(kErrShape, "q2_repack: rows=%d cols=%d (cols a multiple of 64)", rows, cols);
        return 0;
    }
    return repack_mat(static_cast<const uint8_t*>(ggml_rows), rows, cols, static_cast<uint8_t*>(dst));
}

int frt_q2_repack_expert(const void* gate, const void* up, const void* down, int d_model, int d_ff, void* blob) {
    if (!gate || !up || !down || !blob) return set_error(kErrNull, "q2_repack_expert: null pointer");
    if (d_model < kBlock || d_ff < kBlock || d_model % kBlock || d_ff % kBlock)
        return set_error(kErrShape, "q2_repack_expert: d_model=%d d_ff=%d (multiples of 64)", d_model, d_ff);
    uint8_t* p = static_cast<uint8_t*>(blob);
    const size_t gu = mat_bytes(d_ff, d_model);
    repack_mat(static_cast<const uint8_t*>(gate), d_ff, d_model, p);
    repack_mat(static_cast<const uint8_t*>(up), d_ff, d_model, p + gu);
    repack_mat(static_cast<const uint8_t*>(down), d_model, d_ff, p + 2 * gu);
    return kOk;
}

int frt_load_experts(const char* const* shards, int n_shards, const frt_expert_slab* slabs, int d_model, int d_ff,
                     const frt_arena* arena, int threads, frt_load_stats* stats) {
    if (!shards || n_shards < 1 || !slabs || !arena || !arena->base) return set_error(kErrNull, "load_experts: null argument");
    if (arena->blob_bytes != expert_bytes(d_model, d_ff))
        return set_error(kErrShape, "load_experts: the arena's blobs are %zu bytes, the model's experts %zu",
                         arena->blob_bytes, expert_bytes(d_model, d_ff));
    for (int l = 0; l < arena->n_layer; ++l)
        for (int k = 0; k < 3; ++k)
            if (slabs[3 * l + k].shard < 0 || slabs[3 * l + k].shard >= n_shards)
                return set_error(kErrShape, "load_experts: layer %d slab %d names shard %d of %d", l, k, slabs[3 * l + k].shard,
                                 n_shards);
    const int n_layer = arena->n_layer, n_expert = arena->n_expert;
    const size_t slice[3] = {mat_bytes(d_ff, d_model), mat_bytes(d_ff, d_model), mat_bytes(d_model, d_ff)};
    const int per_layer = (n_expert + kExpertsPerItem - 1) / kExpertsPerItem;
    const int n_items = n_layer * per_layer;
    if (threads < 1) threads = 1;
    std::atomic<int> next{0};
    std::atomic<uint64_t> total{0};
    std::mutex err_mu;
    std::string err;
    auto fail = [&](const std::string& m) {
        std::lock_guard<std::mutex> lk(err_mu);
        if (err.empty()) err = m;
        next.store(n_items);
    };
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> pool;
    for (int ti = 0; ti < threads; ++ti) {
        pool.emplace_back([&] {
            std::vector<FdCloser> fds(n_shards);
            for (int i = 0; i < n_shards; ++i) {
                fds[i].fd = open(shards[i], O_RDONLY | O_DIRECT);
                if (fds[i].fd < 0 && errno == EINVAL) fds[i].fd = open(shards[i], O_RDONLY);   // no O_DIRECT here
                if (fds[i].fd < 0) return fail(std::string("open ") + shards[i] + ": " + std::strerror(errno));
            }
            uint8_t* rbuf[3] = {nullptr, nullptr, nullptr};
            size_t rcap[3] = {0, 0, 0};
            uint8_t* stage = nullptr;   // pinned, kExpertsPerItem blobs at the arena's stride
            hipStream_t st = nullptr;
            auto cleanup = [&] {
                for (auto* b : rbuf) std::free(b);
                if (stage) (void)hipHostFree(stage);
                if (st) (void)hipStreamDestroy(st);
            };
            if (hipHostMalloc(reinterpret_cast<void**>(&stage), arena->stride * kExpertsPerItem) != hipSuccess ||
                hipStreamCreate(&st) != hipSuccess) {
                cleanup();
                return fail("load_experts: pinned staging or stream allocation failed");
            }
            uint64_t read = 0;
            for (int it; (it = next.fetch_add(1)) < n_items;) {
                const int l = it / per_layer, e0 = (it % per_layer) * kExpertsPerItem;
                const int ne = n_expert - e0 < kExpertsPerItem ? n_expert - e0 : kExpertsPerItem;
                const uint8_t* src[3];
                bool ok = true;
                for (int k = 0; k < 3 && ok; ++k) {   // aligned pread of [off, off + len)
                    const frt_expert_slab& sl = slabs[3 * l + k];
                    const uint64_t off = sl.file_offset + uint64_t(e0) * slice[k], len = uint64_t(ne) * slice[k];
                    const uint64_t a0 = off & ~uint64_t(kAlign - 1), a1 = (off + len + kAlign - 1) & ~uint64_t(kAlign - 1);
                    if (rcap[k] < a1 - a0) {
                        std::free(rbuf[k]);
                        rbuf[k] = static_cast<uint8_t*>(std::aligned_alloc(kAlign, size_t(a1 - a0)));
                        rcap[k] = rbuf[k] ? size_t(a1 - a0) : 0;
                        if (!rbuf[k]) {
                            ok = false;
                            fail("load_experts: read buffer allocation failed");
                            break;
                        }
                    }
                    size_t done = 0;
                    while (done < a1 - a0) {
                        const ssize_t r = pread(fds[sl.shard].fd, rbuf[k] + done, size_t(a1 - a0 - done), off_t(a0 + done));
                        if (r < 0) {
                            ok = false;
                            fail(std::string("load_experts: pread: ") + std::strerror(errno));
                            break;
                        }
                        if (r == 0) break;   // end of file inside the last aligned block
                        done += size_t(r);
                    }
                    if (ok && done < off - a0 + len) {
                        ok = false;
                        fail("load_experts: short read of an expert slab (layer " + std::to_string(l) + ")");
                    }
                    read += done;
                    src[k] = rbuf[k] + (off - a0);
                }
                if (!ok) break;
                for (int e = 0; e < ne; ++e)
                    frt_q2_repack_expert(src[0] + size_t(e) * slice[0], src[1] + size_t(e) * slice[1],
                                         src[2] + size_t(e) * slice[2], d_model, d_ff, stage + size_t(e) * arena->stride);
                uint8_t* dst = arena->base + (size_t(l) * n_expert + e0) * arena->stride;
                if (hipMemcpyAsync(dst, stage, size_t(ne - 1) * arena->stride + arena->blob_bytes, hipMemcpyHostToDevice, st) !=
                        hipSuccess ||
                    hipStreamSynchronize(st) != hipSuccess) {
                    fail("load_experts: upload to the arena failed");
                    break;
                }
            }
            total += read;
            cleanup();
        });
    }
    for (auto& t : pool) t.join();
    if (!err.empty()) return set_error(kErrIo, "%s", err.c_str());
    if (stats) {
        stats->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        stats->bytes_read = total.load();
    }
    return kOk;
}

}  // extern "C"
