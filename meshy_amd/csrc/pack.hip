// Micro-batch materialisation and GRPO advantages for gfx950.
//
// meshy_pack_micro_batches builds every micro of a rank in two launches:
//   k_pack_scan  one workgroup per micro: a block-wide prefix scan of the
//                micro's document lengths gives cu_seqlens (packed layout,
//                batch.py:154-177), including the padding document;
//   k_pack_fill  one thread per output token: the owning document comes from a
//                binary search in cu_seqlens (packed) or the row index
//                (padded); the token is gathered from the sample's flat
//                buffers with the per-document shift-by-one of labels, mask and
//                rollout logprobs (batch.py:91-93, 126-172), and the position
//                is the offset inside the document.
// meshy_zero_variance_groups flags the groups whose raw rewards are all equal
// (within a tolerance), one wavefront per group.
// meshy_grpo_advantage normalises rewards per group, one wavefront per group
// (rollout.py:88-97).
#include "common.h"

namespace meshy {
namespace {

constexpr int kScanThreads = 256;
constexpr int kFillThreads = 256;
constexpr int kFillItems = 1;  // tokens per thread

// Inclusive block scan of one int64 per thread.
__device__ __forceinline__ int64_t block_inclusive_scan(int64_t v, int64_t* wave_tot) {
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int64_t n = __shfl_up(v, off, kWave);
        if (lane >= off) v += n;
    }
    if (lane == kWave - 1) wave_tot[wid] = v;
    __syncthreads();
    int64_t carry = 0;
    for (int w = 0; w < wid; ++w) carry += wave_tot[w];
    __syncthreads();
    return v + carry;
}

__global__ __launch_bounds__(kScanThreads) void k_pack_scan(const int64_t* __restrict__ micro_seq_len,
                                                            const int32_t* __restrict__ micro_doc_start,
                                                            const int64_t* __restrict__ doc_len,
                                                            int32_t* __restrict__ cu) {
    __shared__ int64_t wave_tot[kScanThreads / kWave];
    const int k = blockIdx.x;
    const int32_t d0 = micro_doc_start[k];
    const int32_t nd = micro_doc_start[k + 1] - d0;
    int32_t* out = cu + d0 + 2 * k;
    if (threadIdx.x == 0) out[0] = 0;
    int64_t carry = 0;
    for (int32_t base = 0; base < nd; base += kScanThreads) {
        const int32_t j = base + threadIdx.x;
        const int64_t len = (j < nd) ? doc_len[d0 + j] : 0;
        const int64_t incl = block_inclusive_scan(len, wave_tot);
        if (j < nd) out[j + 1] = static_cast<int32_t>(carry + incl);
        int64_t tot = 0;
        for (int w = 0; w < kScanThreads / kWave; ++w) tot += wave_tot[w];
        __syncthreads();  // every wave has read wave_tot before the next chunk rewrites it
        carry += tot;
    }
    if (threadIdx.x == 0) {
        const int64_t T = micro_seq_len[k];
        if (T > carry) out[nd + 1] = static_cast<int32_t>(T);
    }
}

// Packed micros with at most kLdsDocs documents scan their offsets in LDS
// inside k_pack_fill; larger ones use k_pack_scan's global table.
constexpr int kLdsDocs = 1024;

template <typename Tok>
__global__ __launch_bounds__(kFillThreads) void k_pack_fill(meshy_pack_args a) {
    __shared__ int32_t s_cu[kLdsDocs + 2];
    __shared__ int64_t wave_tot[kFillThreads / kWave];
    const int k = blockIdx.y;
    const int64_t out0 = a.micro_out_off[k];
    const int64_t n_elems = a.micro_out_off[k + 1] - out0;
    const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * (kFillThreads * kFillItems);
    // Uniform over the workgroup.  Workgroup 0 of every micro stays, even of
    // one without output elements (all its documents empty): it writes the
    // per-document tables.
    if (tile0 >= n_elems && blockIdx.x > 0) return;
    const int64_t S = a.micro_seq_len[k];
    const int32_t d0 = a.micro_doc_start[k];
    const int32_t nd = a.micro_doc_start[k + 1] - d0;
    const Tok* tokens = static_cast<const Tok*>(a.tokens);
    const bool packed = a.layout == MESHY_LAYOUT_PACKED;
    int32_t* cu_out = a.cu_seqlens ? a.cu_seqlens + d0 + 2 * k : nullptr;
    const int32_t* cu = cu_out;
    if (packed && nd <= kLdsDocs) {
        // Exclusive prefix of the document lengths: cu_seqlens (batch.py:154-177).
        int64_t carry = 0;
        for (int32_t base = 0; base < nd; base += kFillThreads) {
            const int32_t j = base + threadIdx.x;
            const int64_t len = (j < nd) ? a.doc_len[d0 + j] : 0;
            const int64_t incl = block_inclusive_scan(len, wave_tot);
            if (j < nd) s_cu[j + 1] = static_cast<int32_t>(carry + incl);
            int64_t tot = 0;
            for (int w = 0; w < kFillThreads / kWave; ++w) tot += wave_tot[w];
            __syncthreads();
            carry += tot;
        }
        if (threadIdx.x == 0) s_cu[0] = 0;
        __syncthreads();
        cu = s_cu;
        if (blockIdx.x == 0) {
            for (int32_t j = threadIdx.x; j <= nd; j += kFillThreads) cu_out[j] = s_cu[j];
            if (threadIdx.x == 0 && S > carry) cu_out[nd + 1] = static_cast<int32_t>(S);
        }
    }

    if (blockIdx.x == 0) {
        for (int32_t j = threadIdx.x; j < nd; j += kFillThreads) {
            if (a.adv_doc) a.adv_doc[d0 + j] = a.adv_samples[a.doc_sample[d0 + j]];
            if (a.doc_len_out) a.doc_len_out[d0 + j] = static_cast<int32_t>(a.doc_len[d0 + j]);
        }
        // Token offsets of the micro's n_docs + 1 document slots over its
        // flattened [rows, S] grid (slot nd, the padding, last): what the loss
        // kernels take as seg_offsets.
        if (a.seg_offsets) {
            int64_t* so = a.seg_offsets + d0 + 2 * k;
            for (int32_t j = threadIdx.x; j <= nd + 1; j += kFillThreads) {
                int64_t v;
                if (packed) v = j <= nd ? static_cast<int64_t>(cu[j]) : S;
                else v = (j <= nd ? min<int64_t>(j, max(nd, 1)) : max(nd, 1)) * S;
                so[j] = v;
            }
        }
    }

#pragma unroll
    for (int it = 0; it < kFillItems; ++it) {
        const int64_t i = tile0 + it * kFillThreads + threadIdx.x;
        if (i >= n_elems) break;
        int32_t d;     // document slot, nd = padding
        int64_t p;     // position inside the document (packed) or row (padded)
        if (packed) {
            // Largest d in [0, nd] with cu[d] <= i.
            int32_t lo = 0, hi = nd;
            while (lo < hi) {
                const int32_t mid = (lo + hi + 1) >> 1;
                if (static_cast<int64_t>(cu[mid]) <= i) lo = mid;
                else hi = mid - 1;
            }
            d = lo;
            p = i - cu[d];
        } else {
            const int64_t row = i / S;
            p = i - row * S;
            d = static_cast<int32_t>(row);
        }
        const int64_t o = out0 + i;
        int64_t in_id = 0, lab = 0;
        float mk = 0.f, lp = 0.f, adv = 0.f;
        const bool real = d < nd && p < a.doc_len[d0 + d];
        int64_t src = -1;
        if (real) {
            const int32_t smp = a.doc_sample[d0 + d];
            const int64_t L = a.doc_len[d0 + d];
            src = a.sample_offsets[smp] + p;
            in_id = static_cast<int64_t>(tokens[src]);
            if (p + 1 < L) {
                lab = static_cast<int64_t>(tokens[src + 1]);
                mk = a.mask_u8 ? static_cast<float>(static_cast<const uint8_t*>(a.mask)[src + 1])
                               : static_cast<const float*>(a.mask)[src + 1];
                if (a.logprobs) lp = a.logprobs[src + 1];
            }
            if (a.adv_tokens) adv = a.adv_tokens[src];
        }
        if (a.adv_tok && !a.adv_tokens && a.adv_samples && d < nd) adv = a.adv_samples[a.doc_sample[d0 + d]];
        a.input_ids[o] = in_id;
        a.labels[o] = lab;
        a.mask_out[o] = mk;
        if (a.rollout_lp) a.rollout_lp[o] = lp;
        if (a.adv_tok) a.adv_tok[o] = adv;
        // Padded: every row of a real micro is its document; a filler's
        // single row is padding slot 0 (batch.py:123, 137-139).
        a.doc_ids[o] = packed ? static_cast<int64_t>(d) : (nd == 0 ? 0 : static_cast<int64_t>(d));
        a.positions[o] = static_cast<int32_t>(p);
        if (a.teacher_k > 0) {
            // Teacher rows are indexed by logits position: no shift (opd.py:58-89).
            const int64_t K = a.teacher_k;
            int64_t* ids_o = a.teacher_ids_out + o * K;
            float* lps_o = a.teacher_lps_out + o * K;
            const bool ids64 = a.teacher_ids_elem_bytes == 8;  // uniform over the launch
            for (int64_t j = 0; j < K; ++j) {
                const int64_t at = src * K + j;
                ids_o[j] = src < 0 ? 0
                           : ids64 ? static_cast<const int64_t*>(a.teacher_ids)[at]
                                   : static_cast<int64_t>(static_cast<const int32_t*>(a.teacher_ids)[at]);
                lps_o[j] = src >= 0 ? a.teacher_lps[src * K + j] : 0.f;
            }
        }
    }
}

// Each group's range is clamped to [0, n_rewards): malformed offsets stay in bounds.
__global__ __launch_bounds__(kWave) void k_grpo(const float* __restrict__ rewards, int64_t n_rewards,
                                                const int64_t* __restrict__ group_off,
                                                float* __restrict__ adv) {
    const int64_t g = blockIdx.x;
    const int64_t b = min(max(group_off[g], static_cast<int64_t>(0)), n_rewards);
    const int64_t n = min(max(group_off[g + 1], b), n_rewards) - b;
    const int lane = threadIdx.x;
    if (n <= 0) return;
    if (n == 1) {
        if (lane == 0) adv[b] = rewards[b];
        return;
    }
    float sum = 0.f;
    for (int64_t i = lane; i < n; i += kWave) sum += rewards[b + i];
    sum = wave_sum(sum);
    const float mean = sum / static_cast<float>(n);
    float sq = 0.f;
    for (int64_t i = lane; i < n; i += kWave) {
        const float dv = rewards[b + i] - mean;
        sq = fmaf(dv, dv, sq);
    }
    sq = wave_sum(sq);
    const float std = sqrtf(sq / static_cast<float>(n - 1));
    const float den = fmaxf(std, 1e-8f);
    for (int64_t i = lane; i < n; i += kWave) adv[b + i] = (rewards[b + i] - mean) / den;
}

// Python's max() and min() over a list start from the first element and take
// a later one only when it compares greater (smaller).  A NaN first element
// therefore stays, and a later NaN never wins.  So a group has zero variance
// when its first raw reward is not NaN and the spread of its non-NaN rewards
// is within the tolerance (inf - inf is NaN: not within).  Empty groups have
// zero variance.  Ranges are clamped to [0, n_raw) as in k_grpo.
__global__ __launch_bounds__(kWave) void k_zero_variance(const double* __restrict__ raw, int64_t n_raw,
                                                         const int64_t* __restrict__ group_off, double tol,
                                                         uint8_t* __restrict__ flags) {
    const int64_t g = blockIdx.x;
    const int64_t b = min(max(group_off[g], static_cast<int64_t>(0)), n_raw);
    const int64_t n = min(max(group_off[g + 1], b), n_raw) - b;
    const int lane = threadIdx.x;
    double hi = -__builtin_inf(), lo = __builtin_inf();
    for (int64_t i = lane; i < n; i += kWave) {
        const double r = raw[b + i];
        hi = r > hi ? r : hi;
        lo = r < lo ? r : lo;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const double h = __shfl_xor(hi, off, kWave);
        const double l = __shfl_xor(lo, off, kWave);
        hi = h > hi ? h : hi;
        lo = l < lo ? l : lo;
    }
    if (lane == 0) flags[g] = n <= 0 ? 1 : static_cast<uint8_t>(!isnan(raw[b]) && hi - lo <= tol);
}

}  // namespace
}  // namespace meshy

extern "C" int meshy_pack_micro_batches(const meshy_pack_args* args, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (!args) return set_error(MESHY_ENULL, "meshy_pack_micro_batches: args is NULL");
    const meshy_pack_args& a = *args;
    if (a.n_micro < 0 || a.n_samples < 0)
        return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: negative counts");
    if (a.n_micro == 0) return MESHY_OK;
    if (a.layout != MESHY_LAYOUT_PADDED && a.layout != MESHY_LAYOUT_PACKED)
        return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: unknown layout %d", a.layout);
    if (a.tokens_elem_bytes != 4 && a.tokens_elem_bytes != 8)
        return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: tokens must be int32 or int64");
    if (!a.micro_seq_len || !a.micro_out_off || !a.micro_doc_start || !a.input_ids || !a.labels ||
        !a.positions || !a.mask_out || !a.doc_ids)
        return set_error(MESHY_ENULL, "meshy_pack_micro_batches: plan tables and outputs are required");
    if (a.max_docs_per_micro > 0 && (!a.tokens || !a.mask || !a.sample_offsets || !a.doc_sample || !a.doc_len))
        return set_error(MESHY_ENULL, "meshy_pack_micro_batches: sample buffers are required");
    if (a.layout == MESHY_LAYOUT_PACKED && !a.cu_seqlens)
        return set_error(MESHY_ENULL, "meshy_pack_micro_batches: packed layout needs cu_seqlens");
    if (a.adv_doc && !a.adv_samples)
        return set_error(MESHY_ENULL, "meshy_pack_micro_batches: adv_doc needs adv_samples");
    if (a.adv_tok && !a.adv_tokens && !a.adv_samples)
        return set_error(MESHY_ENULL, "meshy_pack_micro_batches: adv_tok needs adv_tokens or adv_samples");
    if (a.max_micro_elems < 0 || a.max_micro_elems > INT32_MAX)
        return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: bad max_micro_elems %lld",
                         static_cast<long long>(a.max_micro_elems));
    if (a.n_micro > 65535) return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: too many micros");
    if (a.teacher_k < 0) return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: negative teacher_k");
    if (a.teacher_ids_elem_bytes != 0 && a.teacher_ids_elem_bytes != 4 && a.teacher_ids_elem_bytes != 8)
        return set_error(MESHY_EINVAL, "meshy_pack_micro_batches: teacher ids must be int32 or int64");
    if (a.teacher_k > 0 && (!a.teacher_ids_out || !a.teacher_lps_out ||
                            (a.max_docs_per_micro > 0 && (!a.teacher_ids || !a.teacher_lps))))
        return set_error(MESHY_ENULL, "meshy_pack_micro_batches: teacher columns need inputs and outputs");

    // max_docs_per_micro must bound every micro's document count: micros with
    // more than kLdsDocs documents read the table this launch writes.
    if (a.layout == MESHY_LAYOUT_PACKED && a.max_docs_per_micro > kLdsDocs) {
        hipLaunchKernelGGL(k_pack_scan, dim3(static_cast<unsigned>(a.n_micro)), dim3(kScanThreads), 0, stream,
                           a.micro_seq_len, a.micro_doc_start, a.doc_len, a.cu_seqlens);
        int rc = check_launch("meshy_pack_micro_batches(scan)");
        if (rc) return rc;
    }
    const int64_t per_block = static_cast<int64_t>(kFillThreads) * kFillItems;
    const dim3 grid(static_cast<unsigned>(std::max<int64_t>(1, ceil_div(a.max_micro_elems, per_block))),
                    static_cast<unsigned>(a.n_micro));
    if (a.tokens_elem_bytes == 4) {
        hipLaunchKernelGGL(k_pack_fill<int32_t>, grid, dim3(kFillThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL(k_pack_fill<int64_t>, grid, dim3(kFillThreads), 0, stream, a);
    }
    return check_launch("meshy_pack_micro_batches(fill)");
}

extern "C" int meshy_grpo_advantage(const float* rewards, int64_t n_rewards, const int64_t* group_offsets,
                                    int64_t n_groups, float* advantages, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (n_groups < 0 || n_rewards < 0) return set_error(MESHY_EINVAL, "meshy_grpo_advantage: negative count");
    if (n_groups == 0 || n_rewards == 0) return MESHY_OK;
    if (!rewards || !group_offsets || !advantages)
        return set_error(MESHY_ENULL, "meshy_grpo_advantage: NULL pointer");
    if (n_groups > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_grpo_advantage: too many groups");
    hipLaunchKernelGGL(k_grpo, dim3(static_cast<unsigned>(n_groups)), dim3(kWave), 0, stream, rewards, n_rewards,
                       group_offsets, advantages);
    return check_launch("meshy_grpo_advantage");
}

extern "C" int meshy_zero_variance_groups(const double* raw_rewards, int64_t n_rewards,
                                          const int64_t* group_offsets, int64_t n_groups, double tolerance,
                                          uint8_t* flags, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (n_groups < 0 || n_rewards < 0)
        return set_error(MESHY_EINVAL, "meshy_zero_variance_groups: negative count");
    if (n_groups == 0) return MESHY_OK;
    if ((!raw_rewards && n_rewards > 0) || !group_offsets || !flags)
        return set_error(MESHY_ENULL, "meshy_zero_variance_groups: NULL pointer");
    if (n_groups > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_zero_variance_groups: too many groups");
    hipLaunchKernelGGL(k_zero_variance, dim3(static_cast<unsigned>(n_groups)), dim3(kWave), 0, stream, raw_rewards,
                       n_rewards, group_offsets, tolerance, flags);
    return check_launch("meshy_zero_variance_groups");
}
