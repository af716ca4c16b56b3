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

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace meshy
