// Student Top-K on-policy distillation loss, its sums and its gradient, for gfx950.
//
// Restates StudentTopKTrainer._distill_loss (meshy/backend/titan/opd.py:153-197)
// after the gather, with forward_kl_topk (meshy/backend/titan/topk_loss.py:60-80):
//   log_s = clamp_min(student_k, c), log_t = clamp_min(teacher_k, c)      (74-76)
//   kl    = sum_k exp(log_t) (log_t - log_s), clamped to [-L, L]          (77-79)
//   per-document sums of kl * mask and of mask; token-mean or
//   sequence-mean reduction with global denominators                      (opd.py:168-181)
//   token_count, student / teacher Top-K mass, train-vs-rollout k3 and
//   |logdiff| sums of the sampled token                                   (opd.py:183-196)
//
// Student values come as the [n, K + 1] output of the gather (K Teacher ids
// plus the sampled label, opd.py:156-162); column K is the sampled token's
// log-prob and carries no gradient.
//
// Layout: documents are contiguous token ranges (seg_offsets), and doc_ids
// (non-decreasing) names each token's document.  Tiles of 256 tokens, one per
// thread:
//   k_distill_tiles  per token terms; a wavefront segmented scan plus a
//                    carry over the waves gives each (tile, document) pair's
//                    partial sums, stored at workspace[tile + document]
//                    (collision-free: documents and tiles are both ordered);
//                    the token-level sums reduce per tile in fixed order;
//   k_distill_final  one workgroup: per-document totals in tile order, the
//                    loss and every sum (fixed order, bitwise reproducible);
//   k_distill_bwd    per token, d loss / d student_k as torch autograd gives
//                    it (clamp passes on its closed range).
#include <math.h>

#include "common.h"

namespace meshy {
namespace {

constexpr int kTileTok = 256;
constexpr int kTileWaves = kTileTok / kWave;
constexpr int kFinalThreads = 1024;
constexpr int kTokSums = 5;  // token_count, student mass, teacher mass, k3, |logdiff|
constexpr int kMaxK = 256;

__device__ __forceinline__ float nan_to_num(float x) {
    if (isnan(x)) return 0.f;
    if (isinf(x)) return x > 0 ? 3.40282347e38f : -3.40282347e38f;
    return x;
}
__device__ __forceinline__ float clamp_lo(float x, float lo) { return isnan(x) ? x : (x < lo ? lo : x); }
__device__ __forceinline__ float clamp_rng(float x, float lo, float hi) {
    return isnan(x) ? x : (x < lo ? lo : (x > hi ? hi : x));
}

__host__ __device__ inline int64_t n_tiles(int64_t n) { return (n + kTileTok - 1) / kTileTok; }

struct Ws {
    float* tok;  // [n_tiles][kTokSums]
    float* seg;  // [n_tiles + n_slots][2]: sum of kl * mask, sum of mask
};

size_t ws_bytes(int64_t n_tokens, int64_t n_docs) {
    const int64_t nt = n_tiles(n_tokens);
    return align_up(sizeof(float) * nt * kTokSums, 256) + align_up(sizeof(float) * 2 * (nt + n_docs + 1), 256);
}

Ws ws_of(void* base, int64_t n_tokens) {
    const int64_t nt = n_tiles(n_tokens);
    Ws w;
    w.tok = static_cast<float*>(base);
    w.seg = reinterpret_cast<float*>(static_cast<char*>(base) + align_up(sizeof(float) * nt * kTokSums, 256));
    return w;
}

// Pre-clamp KL of one token (forward_kl_topk before the loss clamp):
// st and te point at its K student and Teacher log-probs.
__device__ __forceinline__ float kl_of(const float* st, const float* te, int K, bool lp_clamp, float lp_min) {
    float kl = 0.f;
    for (int k = 0; k < K; ++k) {
        float ls = st[k], lt = te[k];
        if (lp_clamp) {
            ls = clamp_lo(ls, lp_min);
            lt = clamp_lo(lt, lp_min);
        }
        kl += expf(lt) * (lt - ls);
    }
    return kl;
}

__device__ __forceinline__ float kl_pre(const meshy_distill_args& a, int64_t i) {
    return kl_of(a.student + i * (a.k + 1), a.teacher + i * a.k, static_cast<int>(a.k), a.has_lp_clamp,
                 a.lp_min_clamp);
}

// d kl / d student_k for a token whose KL gradient is g (after the loss clamp).
__device__ __forceinline__ void kl_grad(const float* st, const float* te, int K, bool lp_clamp, float lp_min,
                                        float g, float* go) {
    for (int k = 0; k < K; ++k) {
        float lt = te[k];
        float pass = 1.f;
        if (lp_clamp) {
            lt = clamp_lo(lt, lp_min);
            pass = (st[k] >= lp_min) ? 1.f : 0.f;
        }
        go[k] = -(g * expf(lt)) * pass;
    }
}

// The document of token i, clamped to the slots so that malformed ids stay in bounds.
__device__ __forceinline__ int64_t doc_at(const meshy_distill_args& a, int64_t i) {
    return min(max(a.doc_ids[i], static_cast<int64_t>(0)), a.n_docs);
}

__global__ __launch_bounds__(kTileTok) void k_distill_tiles(meshy_distill_args a, Ws ws) {
    __shared__ float s_tok[kTileWaves][kTokSums];
    __shared__ float s_tail[kTileWaves][2];     // last lane's segmented partials
    __shared__ int64_t s_first[kTileWaves], s_last[kTileWaves];
    const int64_t b = blockIdx.x;
    const int64_t i = b * kTileTok + threadIdx.x;
    const int64_t n_slots = a.n_docs + 1;
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    const bool ok = i < a.n_tokens;

    float klm = 0.f, mk = 0.f;
    float tok[kTokSums] = {0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t d = n_slots + 1;  // past every slot: never merges with a real token
    if (ok) {
        d = doc_at(a, i);
        mk = a.mask[i];
        float kl = kl_pre(a, i);
        if (a.has_loss_clamp) kl = clamp_rng(kl, -a.loss_max_clamp, a.loss_max_clamp);
        klm = kl * mk;
        const float* st = a.student + i * (a.k + 1);
        const float* te = a.teacher + i * a.k;
        float sm = 0.f, tm = 0.f;
        for (int k = 0; k < static_cast<int>(a.k); ++k) {
            sm += expf(st[k]);
            tm += expf(te[k]);
        }
        tok[0] = mk;
        tok[1] = sm * mk;
        tok[2] = tm * mk;
        if (a.rollout_lp) {
            const float sampled = st[a.k];
            const float diff = a.rollout_lp[i] - sampled;
            const float lr = clamp_rng(diff, -10.f, 10.f);
            tok[3] = nan_to_num(expf(lr) - lr - 1.f) * mk;
            tok[4] = nan_to_num(fabsf(diff)) * mk;
        }
    }

    // Segmented inclusive scan of (klm, mk) over runs of equal d in the wave.
    float vs = klm, vc = mk;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const float ps = __shfl_up(vs, off, kWave);
        const float pc = __shfl_up(vc, off, kWave);
        const int64_t pd = __shfl_up(d, off, kWave);
        if (lane >= off && pd == d) {
            vs += ps;
            vc += pc;
        }
    }
    const int64_t d_next = __shfl_down(d, 1, kWave);
    if (lane == kWave - 1) {
        s_tail[wid][0] = vs;
        s_tail[wid][1] = vc;
        s_last[wid] = d;
    }
    if (lane == 0) s_first[wid] = d;
#pragma unroll
    for (int k = 0; k < kTokSums; ++k) tok[k] = wave_sum(tok[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < kTokSums; ++k) s_tok[wid][k] = tok[k];
    }
    __syncthreads();
    // A run ends where the next token (in this tile) has another document.
    const bool run_end = ok && (lane == kWave - 1 ? (wid == kTileWaves - 1 || s_first[wid + 1] != d) : d_next != d);
    if (run_end) {
        // Portions of the run in earlier waves of this tile, nearest first.
        for (int w = wid - 1; w >= 0 && s_last[w] == d; --w) {
            vs += s_tail[w][0];
            vc += s_tail[w][1];
            if (s_first[w] != d) break;
        }
        float* dst = ws.seg + 2 * (b + d);
        dst[0] = vs;
        dst[1] = vc;
    }
    if (threadIdx.x < kTokSums) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kTileWaves; ++w) v += s_tok[w][threadIdx.x];
        ws.tok[b * kTokSums + threadIdx.x] = v;
    }
}

__global__ __launch_bounds__(kFinalThreads) void k_distill_final(meshy_distill_args a, Ws ws, float* __restrict__ out,
                                                                 float* __restrict__ seg_cnt_out) {
    constexpr int kVals = 1 + kTokSums;
    __shared__ double s_red[kFinalThreads / kWave][kVals];
    __shared__ double s_tot[kVals];
    const int64_t n_slots = a.n_docs + 1;
    const int64_t nt = n_tiles(a.n_tokens);
    double v[kVals];
#pragma unroll
    for (int k = 0; k < kVals; ++k) v[k] = 0.0;
    // The first kFinalThreads tiles' token sums load first: they depend on
    // nothing and arrive while the documents' chain runs.
    float tok0[kTokSums];
    // Every lane loads (tile 0 when it has none, then discarded): a load under
    // a per-lane condition compiles to a branch that waits for each load
    // before the next is issued.
    const bool has_tile = threadIdx.x < nt;
    const int64_t tb = has_tile ? threadIdx.x : 0;
#pragma unroll
    for (int k = 0; k < kTokSums; ++k) tok0[k] = 0.f;
    if (nt > 0) {
#pragma unroll
        for (int k = 0; k < kTokSums; ++k) tok0[k] = ws.tok[tb * kTokSums + k];
#pragma unroll
        for (int k = 0; k < kTokSums; ++k) tok0[k] = has_tile ? tok0[k] : 0.f;
    }
    for (int64_t d = threadIdx.x; d < n_slots; d += kFinalThreads) {
        const int64_t lo = a.seg_offsets[d];
        const int64_t hi = a.seg_offsets[d + 1];
        float sum = 0.f, cnt = 0.f;
        if (hi > lo) {
            for (int64_t t = lo / kTileTok; t <= (hi - 1) / kTileTok; ++t) {
                sum += ws.seg[2 * (t + d)];
                cnt += ws.seg[2 * (t + d) + 1];
            }
        }
        if (seg_cnt_out) seg_cnt_out[d] = cnt;
        if (d < a.n_docs) v[0] += a.per_token_loss ? sum : sum / fmaxf(cnt, 1.f);
    }
#pragma unroll
    for (int k = 0; k < kTokSums; ++k) v[1 + k] += tok0[k];
    for (int64_t t = threadIdx.x + kFinalThreads; t < nt; t += kFinalThreads) {
#pragma unroll
        for (int k = 0; k < kTokSums; ++k) v[1 + k] += ws.tok[t * kTokSums + k];
    }
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
#pragma unroll
    for (int k = 0; k < kVals; ++k) v[k] = wave_sum(v[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < kVals; ++k) s_red[wid][k] = v[k];
    }
    __syncthreads();
    if (threadIdx.x < kVals) {
        double s = 0.0;
        for (int w = 0; w < kFinalThreads / kWave; ++w) s += s_red[w][threadIdx.x];
        s_tot[threadIdx.x] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const double* t = s_tot;
        const double den = a.per_token_loss ? static_cast<double>(max<int64_t>(1, a.n_tokens_global))
                                            : static_cast<double>(max<int64_t>(1, a.n_docs_global));
        out[MESHY_DISTILL_LOSS] = static_cast<float>(t[0] / den);
        out[MESHY_DISTILL_TOKEN_COUNT] = static_cast<float>(t[1]);
        out[MESHY_DISTILL_STUDENT_MASS_SUM] = static_cast<float>(t[2]);
        out[MESHY_DISTILL_TEACHER_MASS_SUM] = static_cast<float>(t[3]);
        out[MESHY_DISTILL_TRAIN_ROLLOUT_KL_SUM] = static_cast<float>(t[4]);
        out[MESHY_DISTILL_TRAIN_ROLLOUT_LOGDIFF_ABS_SUM] = static_cast<float>(t[5]);
    }
}

__global__ __launch_bounds__(kTileTok) void k_distill_bwd(meshy_distill_args a, const float* __restrict__ seg_cnt,
                                                          const float* __restrict__ grad_loss,
                                                          float* __restrict__ grad) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kTileTok + threadIdx.x;
    if (i >= a.n_tokens) return;
    const int64_t d = doc_at(a, i);
    float D = 0.f;  // the padding slot is not in the loss
    if (d < a.n_docs)
        D = a.per_token_loss ? 1.f / static_cast<float>(max<int64_t>(1, a.n_tokens_global))
                             : 1.f / (fmaxf(seg_cnt[d], 1.f) * static_cast<float>(max<int64_t>(1, a.n_docs_global)));
    float g = grad_loss[0] * D * a.mask[i];
    if (a.has_loss_clamp) {
        const float kl = kl_pre(a, i);
        if (!(kl >= -a.loss_max_clamp && kl <= a.loss_max_clamp)) g = 0.f;
    }
    float* go = grad + i * (a.k + 1);
    kl_grad(a.student + i * (a.k + 1), a.teacher + i * a.k, static_cast<int>(a.k), a.has_lp_clamp, a.lp_min_clamp,
            g, go);
    go[a.k] = 0.f;
}

// forward_kl_topk alone (topk_loss.py:60-80), one thread per position.
__global__ __launch_bounds__(kTileTok) void k_fkl(const float* __restrict__ student, const float* __restrict__ teacher,
                                                  int64_t n, int K, int lp_clamp, float lp_min, int loss_clamp,
                                                  float loss_max, float* __restrict__ kl) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kTileTok + threadIdx.x;
    if (i >= n) return;
    float v = kl_of(student + i * K, teacher + i * K, K, lp_clamp, lp_min);
    if (loss_clamp) v = clamp_rng(v, -loss_max, loss_max);
    kl[i] = v;
}

__global__ __launch_bounds__(kTileTok) void k_fkl_bwd(const float* __restrict__ student,
                                                      const float* __restrict__ teacher, int64_t n, int K,
                                                      int lp_clamp, float lp_min, int loss_clamp, float loss_max,
                                                      const float* __restrict__ grad_kl,
                                                      float* __restrict__ grad_student) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kTileTok + threadIdx.x;
    if (i >= n) return;
    const float* st = student + i * K;
    const float* te = teacher + i * K;
    float g = grad_kl[i];
    if (loss_clamp) {
        const float v = kl_of(st, te, K, lp_clamp, lp_min);
        if (!(v >= -loss_max && v <= loss_max)) g = 0.f;
    }
    kl_grad(st, te, K, lp_clamp, lp_min, g, grad_student + i * K);
}

int validate(const meshy_distill_args& a, const char* who) {
    if (a.n_tokens < 0 || a.n_docs < 0) return set_error(MESHY_EINVAL, "%s: negative sizes", who);
    if (a.k < 1 || a.k > kMaxK) return set_error(MESHY_EINVAL, "%s: k must be in [1, %d]", who, kMaxK);
    // Without tokens the per-token arrays may be NULL (an empty tensor has no storage).
    if ((a.n_tokens > 0 && (!a.student || !a.teacher || !a.mask || !a.doc_ids)) || !a.seg_offsets)
        return set_error(MESHY_ENULL, "%s: student, teacher, mask, seg_offsets and doc_ids are required", who);
    return MESHY_OK;
}

}  // namespace
}  // namespace meshy

extern "C" size_t meshy_distill_workspace_size(int64_t n_tokens, int64_t n_docs) {
    if (n_tokens < 0 || n_docs < 0) return 0;
    return meshy::ws_bytes(n_tokens, n_docs);
}

extern "C" int meshy_distill_loss_fwd(const meshy_distill_args* args, float* out, float* seg_cnt,
                                      hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_distill_loss_fwd";
    if (!args || !out) return set_error(MESHY_ENULL, "%s: args and out are required", who);
    const meshy_distill_args& a = *args;
    int rc = validate(a, who);
    if (rc) return rc;
    if (!a.workspace || a.workspace_bytes < ws_bytes(a.n_tokens, a.n_docs))
        return set_error(MESHY_ESPACE, "%s: workspace needs %zu bytes", who, ws_bytes(a.n_tokens, a.n_docs));
    const Ws ws = ws_of(a.workspace, a.n_tokens);
    const int64_t nt = n_tiles(a.n_tokens);
    if (nt > 0) {
        hipLaunchKernelGGL(k_distill_tiles, dim3(static_cast<unsigned>(nt)), dim3(kTileTok), 0, stream, a, ws);
        rc = check_launch(who);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_distill_final, dim3(1), dim3(kFinalThreads), 0, stream, a, ws, out, seg_cnt);
    return check_launch(who);
}

extern "C" int meshy_distill_loss_bwd(const meshy_distill_args* args, const float* seg_cnt, const float* grad_loss,
                                      float* grad_student, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_distill_loss_bwd";
    if (!args || !seg_cnt || !grad_loss)
        return set_error(MESHY_ENULL, "%s: args, seg_cnt, grad_loss and grad_student are required", who);
    const meshy_distill_args& a = *args;
    int rc = validate(a, who);
    if (rc) return rc;
    const int64_t nt = n_tiles(a.n_tokens);
    if (nt == 0) return MESHY_OK;
    if (!grad_student)
        return set_error(MESHY_ENULL, "%s: args, seg_cnt, grad_loss and grad_student are required", who);
    hipLaunchKernelGGL(k_distill_bwd, dim3(static_cast<unsigned>(nt)), dim3(kTileTok), 0, stream, a, seg_cnt,
                       grad_loss, grad_student);
    return check_launch(who);
}

extern "C" int meshy_forward_kl_topk(const float* student, const float* teacher, int64_t n, int64_t k,
                                     int32_t has_lp_clamp, float lp_min_clamp, int32_t has_loss_clamp,
                                     float loss_max_clamp, float* kl, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_forward_kl_topk";
    if (n < 0 || k < 1 || k > kMaxK) return set_error(MESHY_EINVAL, "%s: bad sizes n=%lld k=%lld", who,
                                                      static_cast<long long>(n), static_cast<long long>(k));
    if (n == 0) return MESHY_OK;
    if (!student || !teacher || !kl) return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    hipLaunchKernelGGL(k_fkl, dim3(static_cast<unsigned>(n_tiles(n))), dim3(kTileTok), 0, stream, student, teacher,
                       n, static_cast<int>(k), has_lp_clamp, lp_min_clamp, has_loss_clamp, loss_max_clamp, kl);
    return check_launch(who);
}

extern "C" int meshy_forward_kl_topk_bwd(const float* student, const float* teacher, int64_t n, int64_t k,
                                         int32_t has_lp_clamp, float lp_min_clamp, int32_t has_loss_clamp,
                                         float loss_max_clamp, const float* grad_kl, float* grad_student,
                                         hipStream_t stream) {
    using namespace meshy;
    clear_error();
    const char* who = "meshy_forward_kl_topk_bwd";
    if (n < 0 || k < 1 || k > kMaxK) return set_error(MESHY_EINVAL, "%s: bad sizes n=%lld k=%lld", who,
                                                      static_cast<long long>(n), static_cast<long long>(k));
    if (n == 0) return MESHY_OK;
    if (!student || !teacher || !grad_kl || !grad_student) return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    hipLaunchKernelGGL(k_fkl_bwd, dim3(static_cast<unsigned>(n_tiles(n))), dim3(kTileTok), 0, stream, student,
                       teacher, n, static_cast<int>(k), has_lp_clamp, lp_min_clamp, has_loss_clamp, loss_max_clamp,
                       grad_kl, grad_student);
    return check_launch(who);
}
