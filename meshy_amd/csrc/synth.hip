// Counter-based synthetic bf16 logits drawn from N(0, scale^2), bit-identical
// on the device and the host, for gfx950.
//
// Elements 2p and 2p + 1 of a [rows, cols] fill (element k = row * cols +
// col, pair p = k / 2) are the Box-Muller pair of splitmix64's finaliser of
// mix(seed) ^ p, scaled by `scale` and rounded to bf16 (nearest even); the
// fp32 arithmetic is the project's own (synth_math.h), built only from
// correctly rounded adds, multiplies and fused multiply-adds, so a host can
// regenerate any row of a device tensor bit for bit without copying it.  The
// radius uses 32 bits of uniform, so the largest |z| is sqrt(2 ln 2^32) =
// 6.66 standard deviations: about one value in 4e10 of a true normal lies
// beyond it.
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "common.h"
#include "synth_math.h"

namespace meshy {
namespace {

using synth::mix64;
using synth::normal_bf16_pair;

constexpr int kSynthThreads = 256;
constexpr int kSynthItems = 8;  // consecutive elements per thread: one 16-byte store when aligned

// Element k of the fill (one value of its pair).
__host__ __device__ __forceinline__ uint16_t synth_element(uint64_t seed_mixed, uint64_t k, float scale) {
    uint16_t e0, e1;
    normal_bf16_pair(seed_mixed, k >> 1, scale, e0, e1);
    return (k & 1u) ? e1 : e0;
}

// Grid-stride over groups of 8 elements of the [rows, cols] block; a group
// that crosses a row end or an unaligned row goes element by element.
__global__ __launch_bounds__(kSynthThreads) void k_synth(uint16_t* __restrict__ out, int64_t rows, int64_t cols,
                                                         int64_t row_stride, uint64_t seed_mixed, float scale) {
    const int64_t n = rows * cols;
    const int64_t n_groups = (n + kSynthItems - 1) / kSynthItems;
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * kSynthThreads + threadIdx.x; g < n_groups;
         g += static_cast<int64_t>(gridDim.x) * kSynthThreads) {
        const int64_t k0 = g * kSynthItems;
        const int64_t row = k0 / cols;
        const int64_t col = k0 - row * cols;
        uint16_t* dst = out + row * row_stride + col;
        if (col + kSynthItems <= cols && reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
            uint32_t w[kSynthItems / 2];
#pragma unroll
            for (int q = 0; q < kSynthItems / 2; ++q) {  // k0 is even: element pairs are hash pairs
                uint16_t lo, hi;
                normal_bf16_pair(seed_mixed, static_cast<uint64_t>(k0 / 2 + q), scale, lo, hi);
                w[q] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
            }
            *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int e = 0; e < kSynthItems && k0 + e < n; ++e) {
                const int64_t k = k0 + e;
                const int64_t r = k / cols;
                out[r * row_stride + (k - r * cols)] = synth_element(seed_mixed, static_cast<uint64_t>(k), scale);
            }
        }
    }
}

}  // namespace
}  // namespace meshy

extern "C" int meshy_synth_bf16(uint16_t* out, int64_t rows, int64_t cols, int64_t row_stride, uint64_t seed,
                                float scale, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (rows < 0 || cols < 0 || row_stride < cols) return set_error(MESHY_EINVAL, "meshy_synth_bf16: bad shape");
    if (rows == 0 || cols == 0) return MESHY_OK;
    if (!out) return set_error(MESHY_ENULL, "meshy_synth_bf16: out is NULL");
    if (!(scale >= 0.f) || std::isinf(scale)) return set_error(MESHY_EINVAL, "meshy_synth_bf16: bad scale");
    const int64_t n_groups = (rows * cols + kSynthItems - 1) / kSynthItems;
    const int64_t blocks = std::min<int64_t>(65536, (n_groups + kSynthThreads - 1) / kSynthThreads);
    hipLaunchKernelGGL(k_synth, dim3(static_cast<unsigned>(blocks)), dim3(kSynthThreads), 0, stream, out, rows, cols,
                       row_stride, mix64(seed), scale);
    return check_launch("meshy_synth_bf16");
}

extern "C" int meshy_synth_bf16_rows_host(uint16_t* out, const int64_t* row_ids, int64_t n_rows, int64_t cols,
                                          uint64_t seed, float scale) {
    using namespace meshy;
    clear_error();
    if (n_rows < 0 || cols < 0) return set_error(MESHY_EINVAL, "meshy_synth_bf16_rows_host: bad shape");
    if (n_rows == 0 || cols == 0) return MESHY_OK;
    if (!out || !row_ids) return set_error(MESHY_ENULL, "meshy_synth_bf16_rows_host: NULL pointer");
    if (!(scale >= 0.f) || std::isinf(scale)) return set_error(MESHY_EINVAL, "meshy_synth_bf16_rows_host: bad scale");
    for (int64_t i = 0; i < n_rows; ++i)
        if (row_ids[i] < 0) return set_error(MESHY_EINVAL, "meshy_synth_bf16_rows_host: negative row id");
    const uint64_t sm = mix64(seed);
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int64_t n_threads = std::min<int64_t>(std::min<unsigned>(hw, 16u), std::max<int64_t>(1, n_rows));
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t i = r0; i < r1; ++i) {
            const uint64_t base = static_cast<uint64_t>(row_ids[i]) * static_cast<uint64_t>(cols);
            uint16_t* dst = out + i * cols;
            int64_t c = 0;
            if (base & 1u) {  // the row starts on the second value of a pair
                dst[0] = synth_element(sm, base, scale);
                c = 1;
            }
            for (; c + 1 < cols; c += 2) normal_bf16_pair(sm, (base + static_cast<uint64_t>(c)) >> 1, scale, dst[c], dst[c + 1]);
            if (c < cols) dst[c] = synth_element(sm, base + static_cast<uint64_t>(c), scale);
        }
    };
    // Row ranges go to worker threads; a range whose thread fails to start is
    // done by the calling thread, so a refused thread never escapes as an
    // exception.
    const int64_t per = (n_rows + n_threads - 1) / n_threads;
    std::vector<std::thread> pool;
    std::vector<std::pair<int64_t, int64_t>> left;
    pool.reserve(static_cast<size_t>(n_threads));
    left.reserve(static_cast<size_t>(n_threads));
    for (int64_t t = 1; t < n_threads; ++t) {
        const int64_t r0 = t * per, r1 = std::min(n_rows, r0 + per);
        if (r0 >= r1) continue;
        try {
            pool.emplace_back(work, r0, r1);
        } catch (...) {
            left.emplace_back(r0, r1);
        }
    }
    work(0, std::min(n_rows, per));
    for (const auto& rr : left) work(rr.first, rr.second);
    for (auto& th : pool) th.join();
    return MESHY_OK;
}
