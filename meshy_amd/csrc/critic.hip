// Critic-side reductions of the PPO critic path, for gfx950.
//
//   meshy_per_sequence_mean     advantages_to_per_sequence
//                               (meshy/backend/titan/critic/gae.py:296-312):
//                               out[d] = sum_{i in d} x_i m_i / max(sum m_i, 1);
//   meshy_critic_accumulate     Accumulator.update
//                               (meshy/backend/titan/critic/metrics.py:238-275):
//                               with m = (mask > 0), v = values m, r = returns m,
//                               d = v - r, the window sums of m, r, r^2, d, d^2
//                               (fp64) and each row's v-sum / max(m-sum, 1);
//   meshy_critic_window_sums    critic_diagnostics' token-level sums
//                               (meshy/backend/titan/critic/metrics.py:189-217)
//                               with the mask as given, and each row's mean V;
//   meshy_group_gauges          within_prompt_auc and prompt_pearson
//                               (metrics.py:64-118) over a window's rows;
//   meshy_clipped_value_error   clipped_value_error (meshy/backend/titan/vapo.py:35-41)
//   (+ _bwd)                    max((v - t)^2, (o + clamp(v - o, -c, c) - t)^2)
//                               and its gradient as torch autograd gives it
//                               (maximum splits ties 1/2-1/2, clamp passes on
//                               its closed range).
//
// One workgroup per document (per row for the accumulator) strides its tokens
// with coalesced loads and reduces in a fixed order, so results are bitwise
// reproducible; the window sums take a second one-workgroup pass over the rows.
#include <math.h>

#include "common.h"

namespace meshy {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kAccSums = 5;  // m, r, r^2, d, d^2

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

inline bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <typename T>
__device__ __forceinline__ T block_sum_to0(T v, T* scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    if (lane == 0) scratch[wid] = v;
    __syncthreads();
    T r = 0;
    if (threadIdx.x == 0) {
        for (int w = 0; w < kWaves; ++w) r += scratch[w];
    }
    __syncthreads();
    return r;
}

// N block sums at once: thread 0's v[k] receives the sum of v[k] over the
// block, in the order block_sum_to0 takes (the waves' sums in wave order).
template <int N>
__device__ __forceinline__ void block_sums_to0(double (&v)[N], double (&scratch)[N][kWaves]) {
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const double w = wave_sum(v[k]);
        if (lane == 0) scratch[k][wid] = w;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < N; ++k) {
            double r = 0;
            for (int w = 0; w < kWaves; ++w) r += scratch[k][w];
            v[k] = r;
        }
    }
    __syncthreads();
}

// One workgroup per document.  Its tokens from the first multiple of 8 are
// read 8 at a time (two 16-byte loads per stream, two groups of 8 per thread
// in flight); the head before it and the tail after the last whole group of 8
// one by one.
__global__ __launch_bounds__(kThreads) void k_seq_mean(const float* __restrict__ x, const float* __restrict__ mask,
                                                       const int64_t* __restrict__ seg_off, bool vec,
                                                       float* __restrict__ out) {
    __shared__ float s_a[kWaves], s_b[kWaves];
    const int64_t d = blockIdx.x;
    const int64_t lo = seg_off[d], hi = seg_off[d + 1];
    const int64_t body0 = vec ? min((lo + 7) / 8 * 8, hi) : hi;
    const int64_t n8 = (hi - body0) / 8;
    const int64_t body1 = body0 + 8 * n8;
    float sx[2] = {0.f, 0.f}, sm[2] = {0.f, 0.f};
    auto acc8 = [&](int64_t i, int s) {
        const f32x4 m0 = *reinterpret_cast<const f32x4*>(mask + i);
        const f32x4 m1 = *reinterpret_cast<const f32x4*>(mask + i + 4);
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(x + i);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(x + i + 4);
        sx[s] = fmaf(v0.x, m0.x, fmaf(v0.y, m0.y, fmaf(v0.z, m0.z, fmaf(v0.w, m0.w, sx[s]))));
        sx[s] = fmaf(v1.x, m1.x, fmaf(v1.y, m1.y, fmaf(v1.z, m1.z, fmaf(v1.w, m1.w, sx[s]))));
        sm[s] += ((m0.x + m0.y) + (m0.z + m0.w)) + ((m1.x + m1.y) + (m1.z + m1.w));
    };
    int64_t c = threadIdx.x;
    for (; c + kThreads < n8; c += 2 * kThreads) {
        acc8(body0 + 8 * c, 0);
        acc8(body0 + 8 * (c + kThreads), 1);
    }
    if (c < n8) acc8(body0 + 8 * c, 0);
    for (int64_t i = lo + threadIdx.x; i < body0; i += kThreads) {
        sx[1] = fmaf(x[i], mask[i], sx[1]);
        sm[1] += mask[i];
    }
    for (int64_t i = body1 + threadIdx.x; i < hi; i += kThreads) {
        sx[1] = fmaf(x[i], mask[i], sx[1]);
        sm[1] += mask[i];
    }
    const float tx = block_sum_to0(sx[0] + sx[1], s_a);
    const float tm = block_sum_to0(sm[0] + sm[1], s_b);
    if (threadIdx.x == 0) out[d] = tx / fmaxf(tm, 1.f);
}

__device__ __forceinline__ float load_value(const void* v, int bf16, int64_t i) {
    return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(v)[i]) : static_cast<const float*>(v)[i];
}

// One workgroup per row: row sums into part[row][5] (fp64) and row_value[row].
// Each thread sums its ~S/256 elements in fp32 (two interleaved halves for
// latency), the workgroup combines the threads in fp64.
__device__ __forceinline__ void acc_one(float mk, float val, float ret, float (&a)[kAccSums + 1]) {
    const float m = mk > 0.f ? 1.f : 0.f;
    const float v = val * m;
    const float r = ret * m;
    const float dv = v - r;
    a[0] += m;
    a[1] += r;
    a[2] = fmaf(r, r, a[2]);
    a[3] += dv;
    a[4] = fmaf(dv, dv, a[4]);
    a[5] += v;
}

__device__ __forceinline__ void acc_elem(const void* values, int values_bf16, const float* returns,
                                         const float* mask, int64_t i, float (&a)[kAccSums + 1]) {
    acc_one(mask[i], load_value(values, values_bf16, i), returns[i], a);
}


// The 8 elements at i, a multiple of 8: with 16-byte aligned bases every load
// is a 16-byte vector (values: one for bf16, two for fp32).
struct Elems8 {
    f32x4 m0, m1, r0, r1, v0, v1;
};

__device__ __forceinline__ Elems8 load8(const void* values, int values_bf16, const float* returns,
                                        const float* mask, int64_t i) {
    Elems8 e;
    e.m0 = *reinterpret_cast<const f32x4*>(mask + i);
    e.m1 = *reinterpret_cast<const f32x4*>(mask + i + 4);
    e.r0 = *reinterpret_cast<const f32x4*>(returns + i);
    e.r1 = *reinterpret_cast<const f32x4*>(returns + i + 4);
    if (values_bf16) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(values) + i);
        e.v0 = f32x4{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
        e.v1 = f32x4{bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
    } else {
        e.v0 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(values) + i);
        e.v1 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(values) + i + 4);
    }
    return e;
}

__device__ __forceinline__ void acc8(const Elems8& e, float (&a)[kAccSums + 1]) {
    acc_one(e.m0.x, e.v0.x, e.r0.x, a);
    acc_one(e.m0.y, e.v0.y, e.r0.y, a);
    acc_one(e.m0.z, e.v0.z, e.r0.z, a);
    acc_one(e.m0.w, e.v0.w, e.r0.w, a);
    acc_one(e.m1.x, e.v1.x, e.r1.x, a);
    acc_one(e.m1.y, e.v1.y, e.r1.y, a);
    acc_one(e.m1.z, e.v1.z, e.r1.z, a);
    acc_one(e.m1.w, e.v1.w, e.r1.w, a);
}

// One workgroup per row.  The row's elements from the first multiple of 8 are
// read 8 at a time (two groups of 8 per thread in flight); the head before it
// and the tail after the last whole group of 8 element by element.
__global__ __launch_bounds__(kThreads) void k_acc_rows(const void* __restrict__ values, int values_bf16,
                                                       const float* __restrict__ returns,
                                                       const float* __restrict__ mask, int64_t S, bool vec,
                                                       double* __restrict__ part, float* __restrict__ row_value) {
    __shared__ double s_red[kAccSums + 1][kWaves];
    const int64_t row = blockIdx.x;
    const int64_t base = row * S;
    const int64_t end = base + S;
    const int64_t body0 = vec ? min((base + 7) / 8 * 8, end) : end;
    const int64_t n8 = (end - body0) / 8;
    const int64_t body1 = body0 + 8 * n8;
    float a0[kAccSums + 1] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // m, r, r2, d, d2, v
    float a1[kAccSums + 1] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t c = threadIdx.x;
    for (; c + kThreads < n8; c += 2 * kThreads) {
        const Elems8 e0 = load8(values, values_bf16, returns, mask, body0 + 8 * c);
        const Elems8 e1 = load8(values, values_bf16, returns, mask, body0 + 8 * (c + kThreads));
        acc8(e0, a0);
        acc8(e1, a1);
    }
    if (c < n8) acc8(load8(values, values_bf16, returns, mask, body0 + 8 * c), a0);
    for (int64_t j = base + threadIdx.x; j < body0; j += kThreads) acc_elem(values, values_bf16, returns, mask, j, a1);
    for (int64_t j = body1 + threadIdx.x; j < end; j += kThreads) acc_elem(values, values_bf16, returns, mask, j, a1);
    double acc[kAccSums + 1];
#pragma unroll
    for (int k = 0; k <= kAccSums; ++k) acc[k] = static_cast<double>(a0[k]) + static_cast<double>(a1[k]);
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
#pragma unroll
    for (int k = 0; k <= kAccSums; ++k) {
        const double w = wave_sum(acc[k]);
        if (lane == 0) s_red[k][wid] = w;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t[kAccSums + 1];
#pragma unroll
        for (int k = 0; k <= kAccSums; ++k) {
            t[k] = 0.0;
            for (int w = 0; w < kWaves; ++w) t[k] += s_red[k][w];
        }
#pragma unroll
        for (int k = 0; k < kAccSums; ++k) part[row * kAccSums + k] = t[k];
        // _response_mean: v-sum over max(m-sum, 1)
        row_value[row] = static_cast<float>(t[kAccSums] / fmax(t[0], 1.0));
    }
}

// One workgroup: the window sums over rows in row order.
__global__ __launch_bounds__(kThreads) void k_acc_final(const double* __restrict__ part, int64_t rows,
                                                        double* __restrict__ sums) {
    __shared__ double s_red[kAccSums][kWaves];
    double v[kAccSums];
#pragma unroll
    for (int k = 0; k < kAccSums; ++k) v[k] = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += kThreads) {
#pragma unroll
        for (int k = 0; k < kAccSums; ++k) v[k] += part[r * kAccSums + k];
    }
    block_sums_to0(v, s_red);
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < kAccSums; ++k) sums[k] = v[k];
    }
}

__device__ __forceinline__ float clamp_c(float x, float c) { return isnan(x) ? x : (x < -c ? -c : (x > c ? c : x)); }

__device__ __forceinline__ float cve_of(float v, float t, float o, float clip, int has_clip) {
    const float e = v - t;
    float err = e * e;
    if (has_clip) {
        const float c = (o + clamp_c(v - o, clip)) - t;
        err = fmaxf(err, c * c);
        if (isnan(e) || isnan(c)) err = __builtin_nanf("");
    }
    return err;
}

// d err / d v times gi: maximum splits ties 1/2-1/2, clamp passes on [-clip, clip].
__device__ __forceinline__ float cve_grad(float v, float t, float o, float clip, int has_clip, float gi) {
    const float e = v - t;
    if (!has_clip) return gi * (2.f * e);
    const float dlt = v - o;
    const float c = (o + clamp_c(dlt, clip)) - t;
    const float err = e * e, cerr = c * c;
    float ga = 0.f, gc = 0.f;  // shares of the gradient through each branch of maximum
    if (err > cerr) ga = gi;
    else if (err < cerr) gc = gi;
    else {
        ga = 0.5f * gi;
        gc = 0.5f * gi;
    }
    const float pass = (dlt >= -clip && dlt <= clip) ? 1.f : 0.f;
    return ga * (2.f * e) + (gc * (2.f * c)) * pass;
}


// Four consecutive elements per thread: 16-byte loads and stores when the
// arrays are 16-byte aligned and the four are in range, scalar otherwise.
__global__ __launch_bounds__(kThreads) void k_cve_fwd(const float* __restrict__ v, const float* __restrict__ t,
                                                      const float* __restrict__ o, float clip, int has_clip,
                                                      int64_t n, bool vec, float* __restrict__ out) {
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 4;
    if (i0 >= n) return;
    if (vec && i0 + 4 <= n) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(v + i0);
        const f32x4 t4 = *reinterpret_cast<const f32x4*>(t + i0);
        const f32x4 o4 = has_clip ? *reinterpret_cast<const f32x4*>(o + i0) : f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 r;
        r.x = cve_of(v4.x, t4.x, o4.x, clip, has_clip);
        r.y = cve_of(v4.y, t4.y, o4.y, clip, has_clip);
        r.z = cve_of(v4.z, t4.z, o4.z, clip, has_clip);
        r.w = cve_of(v4.w, t4.w, o4.w, clip, has_clip);
        *reinterpret_cast<f32x4*>(out + i0) = r;
        return;
    }
    for (int64_t i = i0; i < min(i0 + 4, n); ++i) out[i] = cve_of(v[i], t[i], has_clip ? o[i] : 0.f, clip, has_clip);
}

// grad_out is read at i * gs: gs = 1 for a dense gradient, 0 for one value
// broadcast to every element (the gradient of a sum or a mean).
__global__ __launch_bounds__(kThreads) void k_cve_bwd(const float* __restrict__ v, const float* __restrict__ t,
                                                      const float* __restrict__ o, float clip, int has_clip,
                                                      int64_t n, bool vec, const float* __restrict__ g, int64_t gs,
                                                      float* __restrict__ gv) {
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 4;
    if (i0 >= n) return;
    if (vec && i0 + 4 <= n) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(v + i0);
        const f32x4 t4 = *reinterpret_cast<const f32x4*>(t + i0);
        const f32x4 o4 = has_clip ? *reinterpret_cast<const f32x4*>(o + i0) : f32x4{0.f, 0.f, 0.f, 0.f};
        const f32x4 g4 = gs ? *reinterpret_cast<const f32x4*>(g + i0) : f32x4{g[0], g[0], g[0], g[0]};
        f32x4 r;
        r.x = cve_grad(v4.x, t4.x, o4.x, clip, has_clip, g4.x);
        r.y = cve_grad(v4.y, t4.y, o4.y, clip, has_clip, g4.y);
        r.z = cve_grad(v4.z, t4.z, o4.z, clip, has_clip, g4.z);
        r.w = cve_grad(v4.w, t4.w, o4.w, clip, has_clip, g4.w);
        *reinterpret_cast<f32x4*>(gv + i0) = r;
        return;
    }
    for (int64_t i = i0; i < min(i0 + 4, n); ++i)
        gv[i] = cve_grad(v[i], t[i], has_clip ? o[i] : 0.f, clip, has_clip, g[i * gs]);
}

// ---------------------------------------------------------- window gauges
// critic_diagnostics' token-level sums (meshy/backend/titan/critic/metrics.py:
// 189-217) with the float mask as given: one workgroup per row, each thread
// accumulating its elements in fp64, then a fixed-order workgroup sum; the
// window takes a second one-workgroup pass over the rows.
constexpr int kCwSums = MESHY_CW_RMIN;  // the summed values; min and max follow

struct CwAcc {
    double a[kCwSums + 1];  // the sums, then sum v m of the row
    float rmin, rmax;       // of r over the selected tokens
};

__device__ __forceinline__ void cw_one(float m, float v, float r, CwAcc& c) {
    const float e = v - r;
    const bool sel = m > 0.f;
    // variance_reduction selects the masked tokens; the loss, the calibration
    // gap and the row mean multiply by the mask.
    c.a[MESHY_CW_SEL] += sel ? 1.0 : 0.0;
    c.a[MESHY_CW_R] += sel ? static_cast<double>(r) : 0.0;
    c.a[MESHY_CW_R2] += sel ? static_cast<double>(r) * r : 0.0;
    c.a[MESHY_CW_D] += sel ? static_cast<double>(e) : 0.0;
    c.a[MESHY_CW_D2] += sel ? static_cast<double>(e) * e : 0.0;
    c.a[MESHY_CW_M] += m;
    c.a[MESHY_CW_E2M] += static_cast<double>(e * e * m);
    c.a[MESHY_CW_EM] += static_cast<double>(e * m);
    c.a[kCwSums] += static_cast<double>(v * m);
    c.rmin = (sel && r < c.rmin) ? r : c.rmin;
    c.rmax = (sel && r > c.rmax) ? r : c.rmax;
}

__device__ __forceinline__ void cw8(const Elems8& e, CwAcc& c) {
    cw_one(e.m0.x, e.v0.x, e.r0.x, c);
    cw_one(e.m0.y, e.v0.y, e.r0.y, c);
    cw_one(e.m0.z, e.v0.z, e.r0.z, c);
    cw_one(e.m0.w, e.v0.w, e.r0.w, c);
    cw_one(e.m1.x, e.v1.x, e.r1.x, c);
    cw_one(e.m1.y, e.v1.y, e.r1.y, c);
    cw_one(e.m1.z, e.v1.z, e.r1.z, c);
    cw_one(e.m1.w, e.v1.w, e.r1.w, c);
}

// The row's elements from the first multiple of 8 are read 8 at a time with
// 16-byte loads (two groups of 8 per thread in flight, as in k_acc_rows); the
// head before it and the tail after the last whole group element by element.
__global__ __launch_bounds__(kThreads) void k_cw_rows(const void* __restrict__ values, int values_bf16,
                                                      const float* __restrict__ returns,
                                                      const float* __restrict__ mask, int64_t S, bool vec,
                                                      double* __restrict__ part, float* __restrict__ row_value) {
    __shared__ double s_red[kCwSums + 1][kWaves];
    __shared__ float s_min[kWaves], s_max[kWaves];
    const int64_t row = blockIdx.x;
    const int64_t base = row * S;
    const int64_t end = base + S;
    const int64_t body0 = vec ? min((base + 7) / 8 * 8, end) : end;
    const int64_t n8 = (end - body0) / 8;
    const int64_t body1 = body0 + 8 * n8;
    CwAcc c;
#pragma unroll
    for (int k = 0; k <= kCwSums; ++k) c.a[k] = 0.0;
    c.rmin = __builtin_inff();
    c.rmax = -__builtin_inff();
    int64_t g = threadIdx.x;
    for (; g + kThreads < n8; g += 2 * kThreads) {
        const Elems8 e0 = load8(values, values_bf16, returns, mask, body0 + 8 * g);
        const Elems8 e1 = load8(values, values_bf16, returns, mask, body0 + 8 * (g + kThreads));
        cw8(e0, c);
        cw8(e1, c);
    }
    if (g < n8) cw8(load8(values, values_bf16, returns, mask, body0 + 8 * g), c);
    for (int64_t j = base + threadIdx.x; j < body0; j += kThreads)
        cw_one(mask[j], load_value(values, values_bf16, j), returns[j], c);
    for (int64_t j = body1 + threadIdx.x; j < end; j += kThreads)
        cw_one(mask[j], load_value(values, values_bf16, j), returns[j], c);
    double (&a)[kCwSums + 1] = c.a;
    float rmin = c.rmin, rmax = c.rmax;
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
#pragma unroll
    for (int k = 0; k <= kCwSums; ++k) {
        const double w = wave_sum(a[k]);
        if (lane == 0) s_red[k][wid] = w;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float lo = __shfl_xor(rmin, off, kWave);
        const float hi = __shfl_xor(rmax, off, kWave);
        rmin = lo < rmin ? lo : rmin;
        rmax = hi > rmax ? hi : rmax;
    }
    if (lane == 0) {
        s_min[wid] = rmin;
        s_max[wid] = rmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t[kCwSums + 1];
        float lo = __builtin_inff(), hi = -__builtin_inff();
#pragma unroll
        for (int k = 0; k <= kCwSums; ++k) {
            t[k] = 0.0;
            for (int w = 0; w < kWaves; ++w) t[k] += s_red[k][w];
        }
        for (int w = 0; w < kWaves; ++w) {
            lo = s_min[w] < lo ? s_min[w] : lo;
            hi = s_max[w] > hi ? s_max[w] : hi;
        }
        double* dst = part + row * MESHY_CW_VALS;
#pragma unroll
        for (int k = 0; k < kCwSums; ++k) dst[k] = t[k];
        dst[MESHY_CW_RMIN] = lo;
        dst[MESHY_CW_RMAX] = hi;
        row_value[row] = static_cast<float>(t[kCwSums] / fmax(t[MESHY_CW_M], 1.0));
    }
}

__global__ __launch_bounds__(kThreads) void k_cw_final(const double* __restrict__ part, int64_t rows,
                                                       double* __restrict__ sums) {
    __shared__ double s_red[kCwSums][kWaves];
    double v[kCwSums];
#pragma unroll
    for (int k = 0; k < kCwSums; ++k) v[k] = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += kThreads) {
#pragma unroll
        for (int k = 0; k < kCwSums; ++k) v[k] += part[r * MESHY_CW_VALS + k];
    }
    block_sums_to0(v, s_red);
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < kCwSums; ++k) sums[k] = v[k];
    }
    // min and max of r over the selected tokens (+inf / -inf when none)
    double lo = __builtin_inf(), hi = -__builtin_inf();
    for (int64_t r = threadIdx.x; r < rows; r += kThreads) {
        const double a = part[r * MESHY_CW_VALS + MESHY_CW_RMIN];
        const double b = part[r * MESHY_CW_VALS + MESHY_CW_RMAX];
        lo = a < lo ? a : lo;
        hi = b > hi ? b : hi;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const double a = __shfl_xor(lo, off, kWave);
        const double b = __shfl_xor(hi, off, kWave);
        lo = a < lo ? a : lo;
        hi = b > hi ? b : hi;
    }
    __shared__ double s_lo[kWaves], s_hi[kWaves];
    if (threadIdx.x % kWave == 0) {
        s_lo[threadIdx.x / kWave] = lo;
        s_hi[threadIdx.x / kWave] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kWaves; ++w) {
            lo = s_lo[w] < lo ? s_lo[w] : lo;
            hi = s_hi[w] > hi ? s_hi[w] : hi;
        }
        sums[MESHY_CW_RMIN] = lo;
        sums[MESHY_CW_RMAX] = hi;
    }
}

// ---------------------------------------------------------- group gauges
// within_prompt_auc (metrics.py:94-118) and prompt_pearson (64-91): one
// wavefront per row i scans every row j of the window (rows arrive in any
// order and group ids are arbitrary), so row i learns its group's sums and
// whether an earlier row shares its group, and, when it is correct, its wins
// against the group's incorrect rows.  part[i] = {2 wins, pairs, first in
// its group, group mean value, group mean reward}.
constexpr int kGaugeVals = 5;

__global__ __launch_bounds__(kWave) void k_group_rows(const float* __restrict__ value,
                                                      const float* __restrict__ reward,
                                                      const int64_t* __restrict__ gid, int64_t n, float thr,
                                                      double* __restrict__ part) {
    const int64_t i = blockIdx.x;
    const int lane = threadIdx.x;
    const int64_t gi = gid[i];
    const float vi = value[i];
    const bool ci = reward[i] >= thr;
    double wins2 = 0.0, pairs = 0.0, sv = 0.0, sr = 0.0, cnt = 0.0;
    bool earlier = false;
    for (int64_t j = lane; j < n; j += kWave) {
        const bool same = gid[j] == gi;
        const float vj = value[j];
        const float rj = reward[j];
        const bool cj = rj >= thr;
        cnt += same ? 1.0 : 0.0;
        sv += same ? static_cast<double>(vj) : 0.0;
        sr += same ? static_cast<double>(rj) : 0.0;
        earlier = earlier || (same && j < i);
        const bool pair = same && ci && !cj;
        pairs += pair ? 1.0 : 0.0;
        // NaN values compare neither greater nor equal: the pair counts, it never wins
        wins2 += pair ? (vi > vj ? 2.0 : (vi == vj ? 1.0 : 0.0)) : 0.0;
    }
    wins2 = wave_sum(wins2);
    pairs = wave_sum(pairs);
    sv = wave_sum(sv);
    sr = wave_sum(sr);
    cnt = wave_sum(cnt);
    const bool any_earlier = __ballot(earlier) != 0;
    if (lane == 0) {
        double* dst = part + i * kGaugeVals;
        dst[0] = wins2;
        dst[1] = pairs;
        dst[2] = any_earlier ? 0.0 : 1.0;
        dst[3] = sv / cnt;  // cnt >= 1: row i is in its own group
        dst[4] = sr / cnt;
    }
}

// One workgroup: the wins, pairs and groups in a fixed order, then Pearson r
// over the groups' means, centred in a second pass as the reference does.
__global__ __launch_bounds__(kThreads) void k_group_final(const double* __restrict__ part, int64_t n,
                                                          double* __restrict__ out) {
    __shared__ double s_red[kWaves];
    double w = 0.0, p = 0.0, g = 0.0, mv = 0.0, mr = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
        const double* q = part + i * kGaugeVals;
        const bool first = q[2] != 0.0;
        w += q[0];
        p += q[1];
        g += q[2];
        mv += first ? q[3] : 0.0;
        mr += first ? q[4] : 0.0;
    }
    w = block_sum_to0(w, s_red);
    p = block_sum_to0(p, s_red);
    __shared__ double s_g, s_mv, s_mr;
    g = block_sum_to0(g, s_red);
    mv = block_sum_to0(mv, s_red);
    mr = block_sum_to0(mr, s_red);
    if (threadIdx.x == 0) {
        s_g = g;
        s_mv = g > 0.0 ? mv / g : 0.0;
        s_mr = g > 0.0 ? mr / g : 0.0;
    }
    __syncthreads();
    const double G = s_g, cv = s_mv, cr = s_mr;
    double xy = 0.0, xx = 0.0, yy = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
        const double* q = part + i * kGaugeVals;
        const bool first = q[2] != 0.0;
        const double dv = first ? q[3] - cv : 0.0;
        const double dr = first ? q[4] - cr : 0.0;
        xy += dv * dr;
        xx += dv * dv;
        yy += dr * dr;
    }
    xy = block_sum_to0(xy, s_red);
    xx = block_sum_to0(xx, s_red);
    yy = block_sum_to0(yy, s_red);
    if (threadIdx.x == 0) {
        const double den = sqrt(xx) * sqrt(yy);
        out[0] = 0.5 * w;
        out[1] = p;
        out[2] = G;
        out[3] = (G < 2.0 || den == 0.0) ? __builtin_nan("") : xy / den;
    }
}

}  // namespace
}  // namespace meshy

extern "C" int meshy_per_sequence_mean(const float* x, const float* mask, const int64_t* seg_offsets,
                                       int64_t n_docs, float* out, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_per_sequence_mean";
    if (n_docs < 0 || n_docs > INT32_MAX) return set_error(MESHY_EINVAL, "%s: bad n_docs", who);
    if (n_docs == 0) return MESHY_OK;
    if (!x || !mask || !seg_offsets || !out) return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    const bool vec = al16(x) && al16(mask);
    hipLaunchKernelGGL(k_seq_mean, dim3(static_cast<unsigned>(n_docs)), dim3(kThreads), 0, stream, x, mask,
                       seg_offsets, vec, out);
    return check_launch(who);
}

extern "C" size_t meshy_critic_accumulate_workspace_size(int64_t rows) {
    return rows < 0 ? 0 : meshy::align_up(sizeof(double) * meshy::kAccSums * static_cast<size_t>(rows), 256);
}

extern "C" int meshy_critic_accumulate(const void* values, int32_t values_bf16, const float* returns,
                                       const float* mask, int64_t rows, int64_t S, double* sums,
                                       float* row_value, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_critic_accumulate";
    if (rows < 0 || S < 0 || rows > INT32_MAX) return set_error(MESHY_EINVAL, "%s: bad shape", who);
    // Rows of no tokens (S == 0) may come with NULL per-token arrays.
    if (!sums || (rows > 0 && !row_value) || (rows * S > 0 && (!values || !returns || !mask)))
        return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    if (workspace_bytes < meshy_critic_accumulate_workspace_size(rows) || (rows > 0 && !workspace))
        return set_error(MESHY_ESPACE, "%s: workspace needs %zu bytes", who,
                         meshy_critic_accumulate_workspace_size(rows));
    double* part = static_cast<double*>(workspace);
    if (rows > 0) {
        const bool vec = al16(values) && al16(returns) && al16(mask);
        hipLaunchKernelGGL(k_acc_rows, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, stream, values,
                           values_bf16, returns, mask, S, vec, part, row_value);
        int rc = check_launch(who);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_acc_final, dim3(1), dim3(kThreads), 0, stream, part, rows, sums);
    return check_launch(who);
}

extern "C" int meshy_clipped_value_error(const float* values, const float* targets, const float* old_values,
                                         int32_t has_clip, float clip, int64_t n, float* out, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_clipped_value_error";
    if (n < 0) return set_error(MESHY_EINVAL, "%s: negative size", who);
    if (n == 0) return MESHY_OK;
    if (!values || !targets || !out || (has_clip && !old_values))
        return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    const bool vec = al16(values) && al16(targets) && al16(out) && (!has_clip || al16(old_values));
    hipLaunchKernelGGL(k_cve_fwd, dim3(static_cast<unsigned>(ceil_div(n, 4 * kThreads))), dim3(kThreads), 0, stream,
                       values, targets, old_values, clip, has_clip, n, vec, out);
    return check_launch(who);
}

extern "C" int meshy_clipped_value_error_bwd(const float* values, const float* targets, const float* old_values,
                                             int32_t has_clip, float clip, int64_t n, const float* grad_out,
                                             int64_t grad_stride, float* grad_values, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_clipped_value_error_bwd";
    if (n < 0) return set_error(MESHY_EINVAL, "%s: negative size", who);
    if (grad_stride != 0 && grad_stride != 1) return set_error(MESHY_EINVAL, "%s: grad_stride must be 0 or 1", who);
    if (n == 0) return MESHY_OK;
    if (!values || !targets || !grad_out || !grad_values || (has_clip && !old_values))
        return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    const bool vec = al16(values) && al16(targets) && al16(grad_values) && (!has_clip || al16(old_values)) &&
                     (grad_stride == 0 || al16(grad_out));
    hipLaunchKernelGGL(k_cve_bwd, dim3(static_cast<unsigned>(ceil_div(n, 4 * kThreads))), dim3(kThreads), 0, stream,
                       values, targets, old_values, clip, has_clip, n, vec, grad_out, grad_stride, grad_values);
    return check_launch(who);
}

extern "C" size_t meshy_critic_window_workspace_size(int64_t rows) {
    return rows < 0 ? 0 : meshy::align_up(sizeof(double) * MESHY_CW_VALS * static_cast<size_t>(rows), 256);
}

extern "C" int meshy_critic_window_sums(const void* values, int32_t values_bf16, const float* returns,
                                        const float* mask, int64_t rows, int64_t S, double* sums,
                                        float* row_value, void* workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_critic_window_sums";
    if (rows < 0 || S < 0 || rows > INT32_MAX) return set_error(MESHY_EINVAL, "%s: bad shape", who);
    // Rows of no tokens (S == 0) may come with NULL per-token arrays.
    if (!sums || (rows > 0 && !row_value) || (rows * S > 0 && (!values || !returns || !mask)))
        return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    if (workspace_bytes < meshy_critic_window_workspace_size(rows) || (rows > 0 && !workspace))
        return set_error(MESHY_ESPACE, "%s: workspace needs %zu bytes", who, meshy_critic_window_workspace_size(rows));
    double* part = static_cast<double*>(workspace);
    if (rows > 0) {
        const bool vec = al16(values) && al16(returns) && al16(mask);
        hipLaunchKernelGGL(k_cw_rows, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, stream, values,
                           values_bf16, returns, mask, S, vec, part, row_value);
        int rc = check_launch(who);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_cw_final, dim3(1), dim3(kThreads), 0, stream, part, rows, sums);
    return check_launch(who);
}

extern "C" size_t meshy_group_gauges_workspace_size(int64_t n) {
    return n < 0 ? 0 : meshy::align_up(sizeof(double) * meshy::kGaugeVals * static_cast<size_t>(n), 256);
}

extern "C" int meshy_group_gauges(const float* row_value, const float* row_reward, const int64_t* group_ids,
                                  int64_t n, float correct_threshold, double* out, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_group_gauges";
    if (n < 0 || n > INT32_MAX) return set_error(MESHY_EINVAL, "%s: bad size", who);
    if (!out || (n > 0 && (!row_value || !row_reward || !group_ids)))
        return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    if (workspace_bytes < meshy_group_gauges_workspace_size(n) || (n > 0 && !workspace))
        return set_error(MESHY_ESPACE, "%s: workspace needs %zu bytes", who, meshy_group_gauges_workspace_size(n));
    double* part = static_cast<double*>(workspace);
    if (n > 0) {
        hipLaunchKernelGGL(k_group_rows, dim3(static_cast<unsigned>(n)), dim3(kWave), 0, stream, row_value,
                           row_reward, group_ids, n, correct_threshold, part);
        int rc = check_launch(who);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_group_final, dim3(1), dim3(kThreads), 0, stream, part, n, out);
    return check_launch(who);
}
