// Shared helpers of libmeshy_amd: error reporting, bf16 conversion, wave and
// block reductions for 64-wide CDNA wavefronts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "host_common.h"

namespace meshy {

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

// fp32 and fp64 sums over the 64 lanes without the LDS crossbar: each 16-lane
// row reduces with DPP rotations (row_ror 8, 4, 2, 1: full-rate adds, a
// balanced tree), then the four row sums are read into scalars and added as
// (r0 + r1) + (r2 + r3).  Every lane gets the total; all 64 lanes must be active.
template <int kCtrl>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xF, 0xF, false);
}
constexpr int kDppRowRor1 = 0x121, kDppRowRor2 = 0x122, kDppRowRor4 = 0x124, kDppRowRor8 = 0x128;
// Whole-wavefront shift: lane l takes lane l - 1's value, lane 0 gets 0.
constexpr int kDppWaveShr1 = 0x138;

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(dpp_i32<kCtrl>(__float_as_int(v)));
}

template <int kCtrl>
__device__ __forceinline__ double dpp_f64(double v) {
    const long long b = __double_as_longlong(v);
    const unsigned lo = static_cast<unsigned>(dpp_i32<kCtrl>(static_cast<int>(b & 0xffffffffll)));
    const unsigned hi = static_cast<unsigned>(dpp_i32<kCtrl>(static_cast<int>(b >> 32)));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ double lane_f64(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(b & 0xffffffffll), lane));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<kDppRowRor8>(v);
    v += dpp_f32<kDppRowRor4>(v);
    v += dpp_f32<kDppRowRor2>(v);
    v += dpp_f32<kDppRowRor1>(v);
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_f64<kDppRowRor8>(v);
    v += dpp_f64<kDppRowRor4>(v);
    v += dpp_f64<kDppRowRor2>(v);
    v += dpp_f64<kDppRowRor1>(v);
    return (lane_f64(v, 0) + lane_f64(v, 16)) + (lane_f64(v, 32) + lane_f64(v, 48));
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
