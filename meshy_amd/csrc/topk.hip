// Teacher Top-K of bf16 logits with their log-probabilities, for gfx950.
//
// Replaces teacher_topk (meshy/backend/titan/topk_loss.py:20-32): per row,
// the K largest logits (indices and values - logsumexp) of the fp32-upcast
// logits, sorted by value, in one streaming pass over the row instead of an
// fp32 copy, a topk and a logsumexp per chunk.
//
// One workgroup per row.  Every lane streams its 16-byte register tiles once
// and updates the online log-sum-exp (rowstream.h).  Each wavefront also keeps
// a running sorted list of its best entries spread over its 64 lanes (lane j
// holds rank j).  The rank K-1 value is the wavefront's threshold: a tile whose
// lane maxima all fall below it costs one compare, otherwise each 16-byte
// chunk whose maximum reaches it offers its elements at or above it to the
// list one at a time (a ballot, then a shift of the lanes below the insertion
// point).  The first tile sets a floor: the K-th largest of the 64 lanes' tile
// maxima (a 64-lane bitonic sort), which K of the wavefront's elements reach,
// so nothing below it is ever offered.  The threshold then climbs towards the
// row's top values and offers become rare.  The waves' lists are merged by
// wave 0.
//
// Order: torch.sort(descending=True, stable=True)'s, which torch.topk
// follows: NaN ranks above every number (+inf included), larger values before
// smaller, and equal values (NaNs among themselves, -0 and +0 alike) by
// smaller index.  A wavefront that has met NaN or +inf (its running sum turns
// NaN) checks its chunks for NaN explicitly from then on, since a chunk's
// fmaxf maximum skips NaN.  Every list update runs with all 64 lanes active:
// loops are wave-uniform and absent elements are masked by a flag.
#include <algorithm>

#include "rowstream.h"

namespace meshy {
namespace {

constexpr int kTopkThreads = 256;
constexpr int kTopkWaves = kTopkThreads / kWave;
// 8 loads in flight per thread for K <= 16 (764 us on [16384, 151936] at K = 8
// against 820 us with 4); 4 above, where the larger list dominates.
constexpr int kTopkUnrollSmallK = 8;
constexpr int kTopkUnrollLargeK = 4;
constexpr int kSmallK = 16;
constexpr int kMaxTopK = kWave;
constexpr int32_t kNoIndex = INT32_MAX;

// (a, ia) ranks before (b, ib): NaN first, then by value descending, ties
// (NaN with NaN included) by index ascending.
__device__ __forceinline__ bool ranks_before(float a, int32_t ia, float b, int32_t ib) {
    const bool na = isnan(a), nb = isnan(b);
    if (na || nb) return na && (!nb || ia < ib);
    return a > b || (a == b && ia < ib);
}

// A candidate that may rank before the threshold value tv: NaN always may, a
// number when it reaches tv.  One unordered compare: with tv NaN it also
// passes numbers, which ranks_before then rejects.
__device__ __forceinline__ bool may_enter(float z, float tv) { return !(z < tv); }

// Whether any of the 8 elements of a 16-byte chunk is NaN.
__device__ __forceinline__ bool chunk_has_nan(const float* z) {
    bool nan = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) nan |= isnan(z[j]);
    return nan;
}

__device__ __forceinline__ float read_lane(float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ int32_t read_lane(int32_t x, int l) { return __builtin_amdgcn_readlane(x, l); }

// A wavefront's sorted list.  (tv, ti) is the threshold a candidate must rank
// before: the entry of rank K-1, or (floor, kNoIndex) while that entry is below
// the floor, a value at least K of the wavefront's elements reach.
struct WaveTop {
    float v = -__builtin_inff();
    int32_t i = kNoIndex;
    float tv = -__builtin_inff();
    int32_t ti = kNoIndex;
    float floor = -__builtin_inff();
};

__device__ __forceinline__ void refresh_threshold(WaveTop& w, int k) {
    w.tv = read_lane(w.v, k - 1);
    w.ti = read_lane(w.i, k - 1);
    if (w.tv < w.floor) {
        w.tv = w.floor;
        w.ti = kNoIndex;
    }
}

// The k-th largest of the 64 lanes' x (NaN counts as -inf): a 64-lane
// bitonic sort, descending, then lane k-1.
__device__ __forceinline__ float kth_largest_lane(float x, int k) {
    const int lane = threadIdx.x % kWave;
    float v = isnan(x) ? -__builtin_inff() : x;
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            const float o = __shfl_xor(v, stride, kWave);
            const bool desc = (lane & size) == 0 || size == kWave;
            const bool lower = (lane & stride) == 0;
            v = (desc == lower) ? fmaxf(v, o) : fminf(v, o);
        }
    }
    return read_lane(v, k - 1);
}

// Inserts the wave-uniform candidate (cv, ci); the entries ranked before it
// form a prefix of the lanes.
__device__ __forceinline__ void top_insert(WaveTop& w, float cv, int32_t ci, int k) {
    const int lane = threadIdx.x % kWave;
    const int pos = __popcll(__ballot(ranks_before(w.v, w.i, cv, ci)));
    // The entries below the insertion point move down one lane: a DPP
    // wavefront shift (one VALU op each) rather than an LDS-crossbar shuffle.
    const float uv = dpp_f32<kDppWaveShr1>(w.v);
    const int32_t ui = dpp_i32<kDppWaveShr1>(w.i);
    if (lane == pos) {
        w.v = cv;
        w.i = ci;
    } else if (lane > pos) {
        w.v = uv;
        w.i = ui;
    }
    refresh_threshold(w, k);
}

// Offers one element per lane (z, where ok); col(l) is lane l's column.
template <class ColF>
__device__ __forceinline__ void top_offer(WaveTop& w, float z, bool ok, int k, ColF col) {
    uint64_t b = __ballot(ok && may_enter(z, w.tv));
    while (b) {
        const int l = __builtin_ctzll(b);
        b &= b - 1;
        const float cv = read_lane(z, l);
        const int32_t ci = col(l);
        if (ranks_before(cv, ci, w.tv, w.ti)) top_insert(w, cv, ci, k);
    }
}

// Merges the waves' lists into wave 0's (call from every thread).
__device__ __forceinline__ void merge_waves(WaveTop& w, int k) {
    __shared__ float s_v[kTopkWaves][kMaxTopK];
    __shared__ int32_t s_i[kTopkWaves][kMaxTopK];
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    if (lane < k) {
        s_v[wid][lane] = w.v;
        s_i[wid][lane] = w.i;
    }
    __syncthreads();
    if (wid == 0) {
        for (int ww = 1; ww < kTopkWaves; ++ww) {
            for (int j = 0; j < k; ++j) {
                const float cv = s_v[ww][j];
                const int32_t ci = s_i[ww][j];
                // Each list is sorted: once an entry misses, the rest miss too.
                if (!ranks_before(cv, ci, w.tv, w.ti)) break;
                top_insert(w, cv, ci, k);
            }
        }
    }
}

// Writes wave 0's list with lse = m + ln s (thread 0 holds the merged m, s).
__device__ __forceinline__ void write_top(const WaveTop& w, float m, float s, int64_t r, int k,
                                          int64_t* __restrict__ ids, float* __restrict__ lps,
                                          float* __restrict__ lse_out) {
    if (threadIdx.x >= kWave) return;
    // torch.logsumexp: NaN for a row holding NaN, whose top entry is then NaN;
    // otherwise +inf for a row whose max is +inf (its candidates' log-probs are
    // then NaN for the +inf logit and -inf for finite ones), where s is NaN.
    const float top = read_lane(w.v, 0);
    const float lse0 = isnan(top) ? top : (m == __builtin_inff()) ? m : fmaf(__log2f(s), kLn2, m);
    const float lse = read_lane(lse0, 0);
    const int lane = threadIdx.x;
    if (lane == 0 && lse_out) lse_out[r] = lse;
    if (lane < k) {
        ids[r * k + lane] = w.i;
        lps[r * k + lane] = w.v - lse;
    }
}

// The row's last rem (< NT * GMAX) 16-byte chunks, from chunk c0, as one tile
// of G = ceil(rem / NT) loads per thread, all in flight together.  Thread
// tid's group g is chunk c0 + tid + g * NT; groups are offered in order of g,
// the order of one chunk per thread per step.
template <int NT, int G, int GMAX>
__device__ __forceinline__ void topk_tail(const v4u* row4, int64_t c0, int64_t rem, int tid, int wave0, int k,
                                          WaveTop& w, float& m, float& s, float& t) {
    if constexpr (G <= GMAX) {
        if (rem > static_cast<int64_t>(G) * NT) {
            topk_tail<NT, G + 1, GMAX>(row4, c0, rem, tid, wave0, k, w, m, s, t);
            return;
        }
        v4u v[G];
        bool ok[G];
        load_tail<NT, G>(row4 + c0, rem, tid, v, ok);
        float z[G * 8];
        unpack(v, z);
        float cm[G];  // per-group maxima, read only where ok
        bool cn[G];   // per-group NaN flags
#pragma unroll
        for (int g = 0; g < G; ++g) {
            cm[g] = z[8 * g];
#pragma unroll
            for (int j = 1; j < 8; ++j) cm[g] = fmaxf(cm[g], z[8 * g + j]);
            cn[g] = chunk_has_nan(z + 8 * g);
        }
        accumulate_masked<false>(z, ok, m, s, t);  // leaves the present groups' z as loaded
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (__ballot(ok[g] && (cn[g] || cm[g] >= w.tv))) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    top_offer(w, z[8 * g + j], ok[g], k, [&](int l) {
                        return static_cast<int32_t>(8 * (c0 + static_cast<int64_t>(g) * NT + wave0 + l) + j);
                    });
                }
            }
        }
    }
}

template <int NT, int U>
__global__ __launch_bounds__(NT) void k_topk_vec(const uint16_t* __restrict__ logits, int64_t T, int64_t V,
                                                 int64_t stride_b, int64_t stride_t, int k,
                                                 int64_t* __restrict__ ids, float* __restrict__ lps,
                                                 float* __restrict__ lse_out) {
    const int64_t r = blockIdx.x;
    const uint16_t* row = row_ptr(logits, r, T, stride_b, stride_t);
    const v4u* row4 = reinterpret_cast<const v4u*>(row);
    const int tid = threadIdx.x;
    const int wave0 = __builtin_amdgcn_readfirstlane(tid - tid % kWave);  // first thread of this wavefront
    float m = kInit, s = 0.f, t = 0.f;
    WaveTop w;
    const int64_t n8 = V >> 3;
    constexpr int64_t kTile = static_cast<int64_t>(NT) * U;
    const int64_t n_full = n8 / kTile;
    for (int64_t it = 0; it < n_full; ++it) {
        const int64_t c0 = it * kTile;
        v4u v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(row4 + c0 + u * NT + tid);
        float z[U * 8];
        unpack(v, z);
        float cm[U];  // per 16-byte chunk maxima
#pragma unroll
        for (int u = 0; u < U; ++u) {
            cm[u] = z[8 * u];
#pragma unroll
            for (int j = 1; j < 8; ++j) cm[u] = fmaxf(cm[u], z[8 * u + j]);
        }
        float tm = cm[0];
#pragma unroll
        for (int u = 1; u < U; ++u) tm = fmaxf(tm, cm[u]);
        accumulate<false>(z, tm, m, s, t);
        if (it == 0) {
            // k lanes hold an element >= the k-th largest lane maximum.
            w.floor = kth_largest_lane(tm, k);
            refresh_threshold(w, k);
        }
        if (__ballot(tm >= w.tv)) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (__ballot(cm[u] >= w.tv)) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        top_offer(w, z[8 * u + j], true, k, [&](int l) {
                            return static_cast<int32_t>(8 * (c0 + u * NT + wave0 + l) + j);
                        });
                    }
                }
            }
        }
    }
    // A lane's running sum is NaN once it has met NaN or +inf.  The chunk
    // maxima above skip NaN, so such a wavefront rebuilds its list from the
    // full tiles with every chunk checked for NaN (rows of ordinary logits
    // never take this).
    if (__ballot(isnan(s))) {
        w = WaveTop();
        for (int64_t c = tid; c < n_full * kTile; c += NT) {
            const v4u v1[1] = {row4[c]};
            float z1[8];
            unpack(v1, z1);
            if (__ballot(chunk_has_nan(z1) || tile_max(z1) >= w.tv)) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    top_offer(w, z1[j], true, k, [&](int l) { return static_cast<int32_t>(8 * (c - tid + wave0 + l) + j); });
                }
            }
        }
    }
    // Remaining 16-byte chunks: one predicated tile.
    const int64_t rem = n8 - n_full * kTile;
    if (rem > 0) topk_tail<NT, 1, U>(row4, n_full * kTile, rem, tid, wave0, k, w, m, s, t);
    // Tail elements when V is not a multiple of 8 (fewer than 8 < NT).
    if (V & 7) {
        const int64_t e = (n8 << 3) + tid;
        const bool ok = e < V;
        const float z = ok ? bf16_to_f32(row[e]) : 0.f;
        accumulate_one(z, ok, m, s, t);
        top_offer(w, z, ok, k, [&](int l) { return static_cast<int32_t>((n8 << 3) + wave0 + l); });
    }
    merge_waves(w, k);
    block_merge<NT>(m, s, t);
    write_top(w, m, s, r, k, ids, lps, lse_out);
}

// Generic path: any alignment and stride, 2-byte loads, 8 per thread per step.
template <int NT>
__global__ __launch_bounds__(NT) void k_topk_any(const uint16_t* __restrict__ logits, int64_t T, int64_t V,
                                                 int64_t stride_b, int64_t stride_t, int k,
                                                 int64_t* __restrict__ ids, float* __restrict__ lps,
                                                 float* __restrict__ lse_out) {
    const int64_t r = blockIdx.x;
    const uint16_t* row = row_ptr(logits, r, T, stride_b, stride_t);
    const int tid = threadIdx.x;
    const int wave0 = __builtin_amdgcn_readfirstlane(tid - tid % kWave);
    float m = kInit, s = 0.f, t = 0.f;
    WaveTop w;
    for (int64_t e0 = 0; e0 < V; e0 += 8 * NT) {
        float z[8];
        bool ok[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t e = e0 + u * NT + tid;
            ok[u] = e < V;
            z[u] = ok[u] ? bf16_to_f32(row[e]) : 0.f;
            accumulate_one(z[u], ok[u], m, s, t);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            top_offer(w, z[u], ok[u], k, [&](int l) { return static_cast<int32_t>(e0 + u * NT + wave0 + l); });
        }
    }
    merge_waves(w, k);
    block_merge<NT>(m, s, t);
    write_top(w, m, s, r, k, ids, lps, lse_out);
}

}  // namespace
}  // namespace meshy

extern "C" int meshy_topk_logprobs(const uint16_t* logits, int64_t rows, int64_t T, int64_t V, int64_t stride_b,
                                   int64_t stride_t, int64_t k, int64_t* ids, float* logprobs, float* lse,
                                   hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_topk_logprobs";
    if (rows < 0 || T < 0 || V <= 0 || stride_b < 0 || stride_t < 0)
        return set_error(MESHY_EINVAL, "%s: bad shape rows=%lld T=%lld V=%lld", who, static_cast<long long>(rows),
                         static_cast<long long>(T), static_cast<long long>(V));
    if (V > INT32_MAX) return set_error(MESHY_EINVAL, "%s: V must fit in int32", who);
    if (k < 1 || k > kMaxTopK || k > V)
        return set_error(MESHY_EINVAL, "%s: k must be in [1, min(%d, V)], got %lld", who, kMaxTopK,
                         static_cast<long long>(k));
    if (T > 0 && rows > INT32_MAX / T) return set_error(MESHY_EINVAL, "%s: too many rows", who);
    const int64_t n = rows * T;
    if (n == 0) return MESHY_OK;  // an empty call: NULL arrays are accepted
    if (!logits || !ids || !logprobs) return set_error(MESHY_ENULL, "%s: logits, ids and logprobs are required", who);
    const dim3 grid(static_cast<unsigned>(n));
    const bool vec = reinterpret_cast<uintptr_t>(logits) % 16 == 0 && stride_b % 8 == 0 && stride_t % 8 == 0;
    if (vec && k <= kSmallK) {
        hipLaunchKernelGGL((k_topk_vec<kTopkThreads, kTopkUnrollSmallK>), grid, dim3(kTopkThreads), 0, stream,
                           logits, T, V, stride_b, stride_t, static_cast<int>(k), ids, logprobs, lse);
    } else if (vec) {
        hipLaunchKernelGGL((k_topk_vec<kTopkThreads, kTopkUnrollLargeK>), grid, dim3(kTopkThreads), 0, stream,
                           logits, T, V, stride_b, stride_t, static_cast<int>(k), ids, logprobs, lse);
    } else {
        hipLaunchKernelGGL((k_topk_any<kTopkThreads>), grid, dim3(kTopkThreads), 0, stream, logits, T, V, stride_b,
                           stride_t, static_cast<int>(k), ids, logprobs, lse);
    }
    return check_launch(who);
}
