// Building blocks of the kernels that stream one row of bf16 logits per
// workgroup: 16-byte register tiles, the online log-sum-exp state and its
// merges, and the block-wide merge for 64-wide wavefronts.
//
// The online state of a row is a triple over the elements seen so far:
//     m = running max of z,
//     s = sum exp(z - m),
//     t = sum exp(z - m) * (z - m) * log2(e)   (only for the entropy)
// updated once per register tile: the tile max first, then one exp2 per
// element.  lse = m + ln s and H = ln 2 * (log2 s - t / s).
#pragma once

#include <hip/hip_bf16.h>

#include "common.h"

namespace meshy {

// Native 4 x u32 vector: what the nontemporal load/store builtins accept.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kInit = -1e30f;  // finite "minus infinity": keeps 0 * d finite
constexpr int64_t kIgnoreIndex = -100;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Merges (m2, s2, t2) into (m, s, t).
__device__ __forceinline__ void merge(float& m, float& s, float& t, float m2, float s2, float t2) {
    const float mn = fmaxf(m, m2);
    const float d1 = (m - mn) * kLog2e;
    const float d2 = (m2 - mn) * kLog2e;
    const float a1 = fast_exp2(d1);
    const float a2 = fast_exp2(d2);
    t = a1 * fmaf(d1, s, t) + a2 * fmaf(d2, s2, t2);
    s = a1 * s + a2 * s2;
    m = mn;
}

// Moves the running max to at least `tm`, rescaling s and t.
__device__ __forceinline__ void raise_max(float& m, float& s, float& t, float tm) {
    const float mn = fmaxf(m, tm);
    const float d = (m - mn) * kLog2e;
    const float a = fast_exp2(d);
    t = a * fmaf(d, s, t);
    s = a * s;
    m = mn;
}

template <int N>
__device__ __forceinline__ void unpack(const v4u (&v)[N], float (&z)[N * 8]) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
        z[8 * u + 0] = bf16_lo(v[u].x);
        z[8 * u + 1] = bf16_hi(v[u].x);
        z[8 * u + 2] = bf16_lo(v[u].y);
        z[8 * u + 3] = bf16_hi(v[u].y);
        z[8 * u + 4] = bf16_lo(v[u].z);
        z[8 * u + 5] = bf16_hi(v[u].z);
        z[8 * u + 6] = bf16_lo(v[u].w);
        z[8 * u + 7] = bf16_hi(v[u].w);
    }
}

template <int K>
__device__ __forceinline__ float tile_max(const float (&z)[K]) {
    float tm = z[0];
#pragma unroll
    for (int i = 1; i < K; ++i) tm = fmaxf(tm, z[i]);
    return tm;
}

// Accumulates a full register tile (every element valid) whose max is tm.
// kEntropy = false leaves t untouched (log-sum-exp only).
template <bool kEntropy, int K>
__device__ __forceinline__ void accumulate(const float (&z)[K], float tm, float& m, float& s, float& t) {
    raise_max(m, s, t, tm);
    const float nm = -m * kLog2e;
    float s0 = 0.f, s1 = 0.f, t0 = 0.f, t1 = 0.f;
#pragma unroll
    for (int i = 0; i < K; i += 2) {
        const float x0 = fmaf(z[i], kLog2e, nm);
        const float x1 = fmaf(z[i + 1], kLog2e, nm);
        const float e0 = fast_exp2(x0);
        const float e1 = fast_exp2(x1);
        s0 += e0;
        s1 += e1;
        if (kEntropy) {
            t0 = fmaf(e0, x0, t0);
            t1 = fmaf(e1, x1, t1);
        }
    }
    s += s0 + s1;
    if (kEntropy) t += t0 + t1;
}

template <bool kEntropy = true, int K>
__device__ __forceinline__ void accumulate(const float (&z)[K], float& m, float& s, float& t) {
    accumulate<kEntropy>(z, tile_max(z), m, s, t);
}

// Accumulates a full tile against the running max m as it stands, without a
// tile max.  Any reference point gives the same lse and entropy (s and t are
// both relative to m), so this is exact as long as the sums stay finite: it
// is taken only when the tile's sum is at most 2^64, i.e. no element exceeds
// m by more than 64 / log2(e) = 44.4.  Otherwise (and for NaN or infinite
// inputs) it returns false with (s, t) untouched, and the caller accumulates
// the tile with its max.  Saves the tile max and the rescale of every tile
// after a lane's first.
template <bool kEntropy, int U>
__device__ __forceinline__ bool accumulate_at(const v4u (&v)[U], float m, float& s, float& t) {
    const float nm = -m * kLog2e;
    float s0 = 0.f, s1 = 0.f, t0 = 0.f, t1 = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float x0 = fmaf(bf16_lo(w[k]), kLog2e, nm);
            const float x1 = fmaf(bf16_hi(w[k]), kLog2e, nm);
            const float e0 = fast_exp2(x0);
            const float e1 = fast_exp2(x1);
            s0 += e0;
            s1 += e1;
            if (kEntropy) {
                t0 = fmaf(e0, x0, t0);
                t1 = fmaf(e1, x1, t1);
            }
        }
    }
    // Both sums are formed before the test and kept or dropped by a select:
    // a branch around the t update would keep every exp of the tile live.
    const float st = s0 + s1;
    const bool ok = st <= 0x1p64f;
    s = ok ? s + st : s;
    if (kEntropy) t = ok ? t + (t0 + t1) : t;
    return ok;
}

// Accumulates a tile in which only the 8-element groups with ok[g] hold
// data; the others are ignored whatever their contents.
template <bool kEntropy, int G>
__device__ __forceinline__ void accumulate_masked(float (&z)[G * 8], const bool (&ok)[G], float& m, float& s,
                                                  float& t) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; ++k) z[8 * g + k] = ok[g] ? z[8 * g + k] : kInit;
    raise_max(m, s, t, tile_max(z));
    const float nm = -m * kLog2e;
    float s0 = 0.f, t0 = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float x = fmaf(z[8 * g + k], kLog2e, nm);
            const float e = ok[g] ? fast_exp2(x) : 0.f;
            s0 += e;
            if (kEntropy) t0 = fmaf(e, x, t0);
        }
    }
    s += s0;
    if (kEntropy) t += t0;
}

// Loads the last rem (<= NT * G) 16-byte chunks of a row, starting at base,
// G per thread, all issued before any is used: thread tid's chunk g is
// tid + g * NT; past rem it reads chunk 0 instead and its ok flag is false.
template <int NT, int G>
__device__ __forceinline__ void load_tail(const v4u* base, int64_t rem, int tid, v4u (&v)[G], bool (&ok)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int64_t c = tid + static_cast<int64_t>(g) * NT;
        ok[g] = c < rem;
        v[g] = __builtin_nontemporal_load(base + (ok[g] ? c : 0));
    }
}

// Accumulates one element that may be absent.
__device__ __forceinline__ void accumulate_one(float z, bool ok, float& m, float& s, float& t) {
    if (!ok) return;
    raise_max(m, s, t, z);
    const float x = (z - m) * kLog2e;
    const float e = fast_exp2(x);
    s += e;
    t = fmaf(e, x, t);
}

// Block-wide merge of the per-lane triples; the result lands in thread 0.
template <int NT>
__device__ __forceinline__ void block_merge(float& m, float& s, float& t) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float m2 = __shfl_xor(m, off, kWave);
        const float s2 = __shfl_xor(s, off, kWave);
        const float t2 = __shfl_xor(t, off, kWave);
        merge(m, s, t, m2, s2, t2);
    }
    if constexpr (NT > kWave) {
        constexpr int kWaves = NT / kWave;
        __shared__ float sm[kWaves], ss[kWaves], st[kWaves];
        const int lane = threadIdx.x % kWave;
        const int wid = threadIdx.x / kWave;
        if (lane == 0) {
            sm[wid] = m;
            ss[wid] = s;
            st[wid] = t;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
            for (int w = 1; w < kWaves; ++w) merge(m, s, t, sm[w], ss[w], st[w]);
        }
    }
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const __hip_bfloat16 a = __float2bfloat16(lo);
    const __hip_bfloat16 b = __float2bfloat16(hi);
    return static_cast<uint32_t>(__bfloat16_as_ushort(a)) |
           (static_cast<uint32_t>(__bfloat16_as_ushort(b)) << 16);
}

// Row r of a [rows, T, V] tensor with element strides (stride_b, stride_t).
__device__ __forceinline__ const uint16_t* row_ptr(const uint16_t* logits, int64_t r, int64_t T,
                                                   int64_t stride_b, int64_t stride_t) {
    const int64_t b = r / T;
    return logits + b * stride_b + (r - b * T) * stride_t;
}

}  // namespace meshy
