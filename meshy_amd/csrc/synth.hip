// Counter-based synthetic bf16 logits, bit-identical on the device and the
// host, for gfx950.
//
// Element k of a [rows, cols] fill (k = row * cols + col) is a pure function
// of (seed, k), so a host can regenerate any row of a device tensor without
// copying it:
//   h = mix(mix(seed) ^ k)               mix = splitmix64's finaliser
//                                        (Steele, Lea, Flood 2014)
//   s = h[0:16] + h[16:32] + h[32:48] + h[48:64]      four 16-bit uniforms
//   x = (float(s) - 131070) * (scale * sqrt(3) / 65536)    fp32
//   out = bf16(x), rounded to nearest even
// s is an Irwin-Hall sum of four uniforms: mean 0 and standard deviation
// scale (to within 2^-33 relative) after the shift and scale, bounded at
// +-sqrt(3) * 2 * scale.  Only integer operations, one exact conversion, one
// exact subtraction and one rounded multiply touch the value, so both sides
// give the same bits.
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "common.h"

namespace meshy {
namespace {

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__host__ __device__ __forceinline__ uint16_t synth_bf16(uint64_t seed_mixed, uint64_t k, float mult) {
    const uint64_t h = mix64(seed_mixed ^ k);
    const uint32_t s = static_cast<uint32_t>(h & 0xFFFFu) + static_cast<uint32_t>((h >> 16) & 0xFFFFu) +
                       static_cast<uint32_t>((h >> 32) & 0xFFFFu) + static_cast<uint32_t>(h >> 48);
    const float x = (static_cast<float>(s) - 131070.0f) * mult;
    uint32_t u = __builtin_bit_cast(uint32_t, x);  // finite by construction
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// The multiplier, computed once on the host in double and rounded to fp32.
float synth_mult(float scale) { return static_cast<float>(static_cast<double>(scale) * std::sqrt(3.0) / 65536.0); }

constexpr int kSynthThreads = 256;
constexpr int kSynthItems = 8;  // consecutive elements per thread: one 16-byte store when aligned

// Grid-stride over groups of 8 elements of the [rows, cols] block; a group
// that crosses a row end or an unaligned row goes element by element.
__global__ __launch_bounds__(kSynthThreads) void k_synth(uint16_t* __restrict__ out, int64_t rows, int64_t cols,
                                                         int64_t row_stride, uint64_t seed_mixed, float mult) {
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
            for (int q = 0; q < kSynthItems / 2; ++q) {
                const uint32_t lo = synth_bf16(seed_mixed, static_cast<uint64_t>(k0 + 2 * q), mult);
                const uint32_t hi = synth_bf16(seed_mixed, static_cast<uint64_t>(k0 + 2 * q + 1), mult);
                w[q] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int e = 0; e < kSynthItems && k0 + e < n; ++e) {
                const int64_t k = k0 + e;
                const int64_t r = k / cols;
                out[r * row_stride + (k - r * cols)] = synth_bf16(seed_mixed, static_cast<uint64_t>(k), mult);
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
                       row_stride, mix64(seed), synth_mult(scale));
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
    const float mult = synth_mult(scale);
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int64_t n_threads = std::min<int64_t>(std::min<unsigned>(hw, 64u), std::max<int64_t>(1, n_rows));
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t i = r0; i < r1; ++i) {
            const uint64_t base = static_cast<uint64_t>(row_ids[i]) * static_cast<uint64_t>(cols);
            uint16_t* dst = out + i * cols;
            for (int64_t c = 0; c < cols; ++c) dst[c] = synth_bf16(sm, base + static_cast<uint64_t>(c), mult);
        }
    };
    std::vector<std::thread> pool;
    const int64_t per = (n_rows + n_threads - 1) / n_threads;
    for (int64_t t = 1; t < n_threads; ++t) {
        const int64_t r0 = t * per, r1 = std::min(n_rows, r0 + per);
        if (r0 < r1) pool.emplace_back(work, r0, r1);
    }
    work(0, std::min(n_rows, per));
    for (auto& th : pool) th.join();
    return MESHY_OK;
}
