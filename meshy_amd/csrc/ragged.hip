// Token-level rollout statistics over the jagged sample columns, for gfx950.
//
// Replaces the per-token Python loops of TitanTrainer._rollout_metrics
// (meshy/backend/titan/metrics.py:171-322, lines 197-212): per sample the
// response length #(mask > 0), the behaviour-policy log-probs of the sampled
// (mask > 0) tokens -- all of them when the sample's log-prob column is not
// as long as its mask -- their sum, and the kept log-probs themselves, in
// sample order, for the histogram.
//
// Samples are jagged: sample s covers mask[off[s] .. off[s+1]) and
// logprobs[lp_off[s] .. lp_off[s+1]), the values()/offsets() of the rollout's
// jagged nested columns.  Three launches:
//   k_rs_count    one workgroup per sample: counts and the fp64 log-prob sum;
//   k_rs_scan     one workgroup: exclusive scan of the kept counts;
//   k_rs_compact  one workgroup per sample: an ordered stream compaction
//                 (block prefix scan of the keep flags, 1024 tokens per step).
#include "common.h"

namespace meshy {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kScanThreads = 1024;

// Each thread takes kUnroll tokens of a step of kStep (token base + u * kThreads
// + tid): their loads are issued together, so a sample of up to kStep tokens
// costs one memory round trip instead of one per strided iteration.
constexpr int kUnroll = 4;
constexpr int64_t kStep = static_cast<int64_t>(kThreads) * kUnroll;

__global__ __launch_bounds__(kThreads) void k_rs_count(const float* __restrict__ mask,
                                                       const float* __restrict__ lp,
                                                       const int64_t* __restrict__ off,
                                                       const int64_t* __restrict__ lp_off,
                                                       int64_t* __restrict__ resp_len,
                                                       int64_t* __restrict__ kept,
                                                       double* __restrict__ lp_sum) {
    __shared__ int64_t s_c[kWaves], s_k[kWaves];
    __shared__ double s_s[kWaves];
    const int64_t s = blockIdx.x;
    const int64_t m0 = off[s], mn = off[s + 1] - m0;
    const int64_t l0 = lp ? lp_off[s] : 0, ln = lp ? lp_off[s + 1] - l0 : 0;
    // Log-probs are kept where the mask is on when both columns are equally
    // long, else all of them.
    const bool masked = lp && ln == mn;
    int c = 0, k = 0;
    double sum = 0.0;
    // Loads take a clamped index and every one is issued; the out-of-range
    // ones are discarded by a select.  (A load under `j < mn ? ... : 0` becomes
    // a branch that waits for each load before the next.)
    if (masked) {
        for (int64_t base = 0; base < mn; base += kStep) {
            float mv[kUnroll], lv[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t j = min(base + u * kThreads + threadIdx.x, mn - 1);
                mv[u] = mask[m0 + j];
                lv[u] = lp[l0 + j];
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const bool on = base + u * kThreads + threadIdx.x < mn && mv[u] > 0.f;
                c += on;
                k += on;
                sum += on ? static_cast<double>(lv[u]) : 0.0;
            }
        }
    } else {
        for (int64_t base = 0; base < mn; base += kStep) {
            float mv[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) mv[u] = mask[m0 + min(base + u * kThreads + threadIdx.x, mn - 1)];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) c += base + u * kThreads + threadIdx.x < mn && mv[u] > 0.f;
        }
        for (int64_t base = 0; base < ln; base += kStep) {
            float lv[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) lv[u] = lp[l0 + min(base + u * kThreads + threadIdx.x, ln - 1)];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                sum += base + u * kThreads + threadIdx.x < ln ? static_cast<double>(lv[u]) : 0.0;
        }
    }
    const int64_t cw = wave_sum(static_cast<int64_t>(c));
    const int64_t kw = wave_sum(static_cast<int64_t>(k));
    sum = wave_sum(sum);
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    if (lane == 0) {
        s_c[wid] = cw;
        s_k[wid] = kw;
        s_s[wid] = sum;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t tc = 0, tk = 0;
        double ts = 0.0;
        for (int w = 0; w < kWaves; ++w) {
            tc += s_c[w];
            tk += s_k[w];
            ts += s_s[w];
        }
        resp_len[s] = tc;
        kept[s] = masked ? tk : ln;  // ln is 0 without log-probs
        lp_sum[s] = ts;
    }
}

// Exclusive scan of kept[0..n) into out_off[0..n] by one workgroup.
__global__ __launch_bounds__(kScanThreads) void k_rs_scan(const int64_t* __restrict__ kept, int64_t n,
                                                          int64_t* __restrict__ out_off) {
    __shared__ int64_t s_w[kScanThreads / kWave];
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    int64_t carry = 0;
    for (int64_t base = 0; base < n; base += kScanThreads) {
        const int64_t i = base + threadIdx.x;
        int64_t v = i < n ? kept[i] : 0;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const int64_t u = __shfl_up(v, o, kWave);
            if (lane >= o) v += u;
        }
        if (lane == kWave - 1) s_w[wid] = v;
        __syncthreads();
        int64_t before = 0, total = 0;
        for (int w = 0; w < kScanThreads / kWave; ++w) {
            if (w < wid) before += s_w[w];
            total += s_w[w];
        }
        if (i < n) out_off[i + 1] = carry + before + v;
        carry += total;
        __syncthreads();  // s_w is rewritten by the next step
    }
    if (threadIdx.x == 0) out_off[0] = 0;
}

// Ordered compaction of one sample's kept log-probs, kStep tokens per step:
// the kUnroll sub-steps' keep flags are balloted per wave, their popcounts
// exchanged through LDS with one barrier, and each kept value written at
// (tokens kept before its sub-step) + (waves before it) + (lanes before it).
__global__ __launch_bounds__(kThreads) void k_rs_compact(const float* __restrict__ mask,
                                                         const float* __restrict__ lp,
                                                         const int64_t* __restrict__ off,
                                                         const int64_t* __restrict__ lp_off,
                                                         const int64_t* __restrict__ out_off,
                                                         float* __restrict__ out) {
    __shared__ int s_w[2][kUnroll][kWaves];
    const int64_t s = blockIdx.x;
    const int64_t m0 = off[s], mn = off[s + 1] - m0;
    const int64_t l0 = lp_off[s], ln = lp_off[s + 1] - l0;
    const bool masked = ln == mn;
    // The keep flags' source: the mask, or (all kept) the log-probs themselves
    // as a stand-in that is always in range, so the loop has no branch.
    const float* keep_src = masked ? mask + m0 : lp + l0;
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    int64_t dst = out_off[s];
    int buf = 0;
    for (int64_t base = 0; base < ln; base += kStep, buf ^= 1) {
        bool f[kUnroll];
        float lv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            // Clamped indices: every load is issued before any is used.
            const int64_t j = base + u * kThreads + threadIdx.x;
            const int64_t jc = min(j, ln - 1);
            lv[u] = lp[l0 + jc];
            const float mk = keep_src[jc];
            f[u] = (j < ln) & (!masked | (mk > 0.f));  // no short circuit: no branch
        }
        int before_lane[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t b = __ballot(f[u]);
            before_lane[u] = __popcll(b & below);
            if (lane == 0) s_w[buf][u][wid] = __popcll(b);
        }
        // Two LDS buffers alternate between steps, so one barrier per step
        // keeps a fast wave from overwriting counts another still reads.
        __syncthreads();
        int64_t at = dst;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            int before_wave = 0, total = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const int cw = s_w[buf][u][w];
                before_wave += w < wid ? cw : 0;
                total += cw;
            }
            if (f[u]) out[at + before_wave + before_lane[u]] = lv[u];
            at += total;
        }
        dst = at;
    }
}

}  // namespace
}  // namespace meshy

extern "C" size_t meshy_ragged_token_stats_workspace_size(int64_t n) {
    return n < 0 ? 0 : meshy::align_up(sizeof(int64_t) * static_cast<size_t>(n), 256);
}

extern "C" int meshy_ragged_token_stats(const float* mask, const float* logprobs, const int64_t* offsets,
                                        const int64_t* lp_offsets, int64_t n, int64_t* resp_len, double* lp_sum,
                                        int64_t* out_off, float* kept_lp, void* workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_ragged_token_stats";
    if (n < 0 || n > INT32_MAX) return set_error(MESHY_EINVAL, "%s: bad sample count", who);
    if (!out_off) return set_error(MESHY_ENULL, "%s: out_off is required", who);
    if (n > 0 && (!mask || !offsets || !resp_len || !lp_sum))
        return set_error(MESHY_ENULL, "%s: mask, offsets, resp_len and lp_sum are required", who);
    if (logprobs && !lp_offsets) return set_error(MESHY_ENULL, "%s: logprobs need lp_offsets", who);
    if (workspace_bytes < meshy_ragged_token_stats_workspace_size(n) || (n > 0 && !workspace))
        return set_error(MESHY_ESPACE, "%s: workspace needs %zu bytes", who,
                         meshy_ragged_token_stats_workspace_size(n));
    int64_t* kept = static_cast<int64_t*>(workspace);
    if (n > 0) {
        hipLaunchKernelGGL(k_rs_count, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, stream, mask, logprobs,
                           offsets, lp_offsets, resp_len, kept, lp_sum);
        int rc = check_launch(who);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_rs_scan, dim3(1), dim3(kScanThreads), 0, stream, kept, n, out_off);
    int rc = check_launch(who);
    if (rc || n == 0 || !logprobs || !kept_lp) return rc;
    hipLaunchKernelGGL(k_rs_compact, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, stream, mask, logprobs,
                       offsets, lp_offsets, out_off, kept_lp);
    return check_launch(who);
}
