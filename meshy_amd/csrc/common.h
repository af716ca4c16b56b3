// Shared helpers of libmeshy_amd: error reporting, bf16 conversion, wave and
// block reductions for 64-wide CDNA wavefronts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/meshy_amd.h"

namespace meshy {

// Records `msg` (printf-style) as the calling thread's last error and returns code.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Checks the launch that was just enqueued; maps a HIP error to its positive code.
int check_launch(const char* what);

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, kWave));
    return v;
}

// Sums `v` over a block of NT threads; the result is valid in every thread.
// `scratch` holds NT/64 values of T.
template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
    constexpr int kWaves = NT / kWave;
    v = wave_sum(v);
    if constexpr (kWaves == 1) {
        return v;
    } else {
        const int lane = threadIdx.x % kWave;
        const int wid = threadIdx.x / kWave;
        __syncthreads();
        if (lane == 0) scratch[wid] = v;
        __syncthreads();
        T r = scratch[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) r += scratch[w];
        return r;
    }
}

// Largest d in [0, n_slots] with off[d] <= i (off has n_slots + 1 entries,
// non-decreasing): the document slot owning token i.
__device__ __forceinline__ int64_t doc_of(const int64_t* off, int64_t n_slots, int64_t i) {
    int64_t lo = 0, hi = n_slots;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (off[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// doc_of restricted to [lo, hi] (off[lo] <= i): a few steps when the range is
// the handful of documents one tile touches.
__device__ __forceinline__ int64_t doc_of_range(const int64_t* off, int64_t lo, int64_t hi, int64_t i) {
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (off[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// doc_of by one whole wavefront (every lane calls it, the result is uniform):
// a 64-ary search, each round probes 64 evenly spaced slots with one load per
// lane and keeps the bracket of the last slot <= i, so 4096 slots take 2
// dependent loads instead of 12.
__device__ __forceinline__ int64_t doc_of_wave(const int64_t* off, int64_t n_slots, int64_t i) {
    const int lane = threadIdx.x % kWave;
    int64_t lo = 0, hi = n_slots;  // invariant: off[lo] <= i, answer in [lo, hi]
    while (lo < hi) {
        const int64_t span = hi - lo;
        const int64_t p = lo + (span * lane + (kWave - 1)) / kWave;
        const uint64_t b = __ballot(off[p] <= i);  // a prefix of the lanes, lane 0 included
        const int L = kWave - 1 - __clzll(b);
        const int64_t pl = lo + (span * L + (kWave - 1)) / kWave;
        hi = (L == kWave - 1) ? hi : lo + (span * (L + 1) + (kWave - 1)) / kWave - 1;
        lo = pl;
    }
    return lo;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace meshy
