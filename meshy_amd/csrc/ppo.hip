// Token-level clipped PPO loss, its diagnostics and its gradient, for gfx950.
//
// Restates TitanTrainer._ppo_clip_loss (meshy/backend/titan/trainer.py:705-848):
//   r   = exp(new - old)
//   pg  = -min(r*A, clamp(r, 1-eps_lo, 1+eps_hi)*A)                  (760-764)
//   IcePop: w = exp(old - rollout); pg = where(lo<=w<=hi, pg, 0) * w    (766-772)
//   TIS:    pg = where(lo<=r<=hi, pg, 0)                                (773-776)
//   pg *= mask; positive = -new * w_doc * mask                          (777-785)
//   per-document sums, token-mean or sequence-mean reduction            (787-809)
//   diagnostic sums (ratio, clip, KL, ESS, k3, entropy)                 (813-847)
//
// Layout: documents are contiguous token ranges given by seg_offsets
// (non-decreasing doc_ids, the ids the offsets were built from).  The token
// axis is cut into tiles of kTile tokens, one workgroup each.  A tile's
// document range is doc_ids at its two ends; the boundaries between those
// documents are read from seg_offsets, so the per-token ids are never loaded.
// A tile usually overlaps one to four documents: then every thread strides the
// whole tile (coalesced) and accumulates into up to kFastDocs per-document
// slots, reduced once per workgroup.  A tile crossing more documents falls back
// to one wavefront per (tile, document) pair.  Both tiles and documents are ordered,
// so the overlapping pairs form a monotone staircase and `tile + document`
// indexes them without collision.
//   k_ppo_tiles  5 per-document partial sums per pair -> workspace[tile+doc],
//                10 token-level partial sums per tile; with the token-mean
//                reduction also each token's gradient at unit loss gradient;
//   k_ppo_combine one workgroup: per-document totals in tile order, then the
//                loss, ESS and every diagnostic in one fused block reduction
//                (fixed order, no atomics: bitwise reproducible);
//   k_ppo_scale  token mean: d(total loss)/d new_lp = grad_loss * unit gradient;
//   k_ppo_bwd    sequence mean: per token (4 per thread) d(total loss)/d new_lp
//                as torch autograd gives it (min splits ties 1/2-1/2, clamp
//                passes on [lo, hi]), the document's factors gathered by doc_ids.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace meshy {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int64_t kTile = 2048;
constexpr int kFastDocs = 4;  // documents per tile handled by the whole workgroup
constexpr int kTokSums = 10;  // token-level sums
constexpr int kSegSums = 5;   // per-document sums: pg, cnt, w, w2, positive
constexpr int kFinalVals = 4 + kTokSums;

enum TokSum { TS_TIS = 0, TS_RATIO, TS_CLIP, TS_TIS_MASKED, TS_COUNT, TS_KL, TS_LR_ABS, TS_K3, TS_LOGDIFF, TS_ENT };

struct Workspace {
    float* tok;  // [n_tiles][kTokSums]
    float* seg;  // [n_tiles + n_slots][kSegSums]
};

__host__ __device__ inline int64_t n_tiles_of(int64_t n) { return (n + kTile - 1) / kTile; }

size_t ws_bytes(int64_t n_tokens, int64_t n_docs) {
    const int64_t nt = n_tiles_of(n_tokens);
    return align_up(sizeof(float) * nt * kTokSums, 256) + align_up(sizeof(float) * (nt + n_docs + 1) * kSegSums, 256);
}

Workspace ws_of(void* base, int64_t n_tokens) {
    const int64_t nt = n_tiles_of(n_tokens);
    char* p = static_cast<char*>(base);
    Workspace w;
    w.tok = reinterpret_cast<float*>(p);
    w.seg = reinterpret_cast<float*>(p + align_up(sizeof(float) * nt * kTokSums, 256));
    return w;
}

// torch semantics: NaN propagates through min and clamp.
__device__ __forceinline__ float t_min(float a, float b) {
    if (isnan(a) || isnan(b)) return __builtin_nanf("");
    return a < b ? a : b;
}
__device__ __forceinline__ float t_clamp(float x, float lo, float hi) {
    if (isnan(x)) return x;
    return x < lo ? lo : (x > hi ? hi : x);
}
__device__ __forceinline__ float nan_to_num(float x) {
    if (isnan(x)) return 0.f;
    if (isinf(x)) return x > 0 ? 3.40282347e38f : -3.40282347e38f;
    return x;
}

// Per-token forward terms and every per-token sum contribution.
struct Contrib {
    float seg[kSegSums];
    float tok[kTokSums];
};

// The per-token inputs, loaded ahead of the arithmetic.
struct TokIn {
    float nw, ol, mk, ro, en, ad;
};

// kLean: no rollout log-probs, entropy or per-token advantages (the common
// configuration), so only new, old and mask are read and held.
// A lane past the end (!ok) reads token 0 and zeroes the values: loads under a
// per-lane condition compile to branches, and arithmetic on a loaded value
// inside such a branch to a wait per load.  Callers run with n_tokens >= 1.
template <bool kLean = false>
__device__ __forceinline__ TokIn load_tok(const meshy_ppo_args& a, int64_t i, bool ok) {
    const int64_t j = ok ? i : 0;
    TokIn x;
    x.nw = a.new_lp[j];
    x.ol = a.old_lp[j];
    x.mk = a.mask[j];
    x.ro = (!kLean && a.rollout_lp) ? a.rollout_lp[j] : 0.f;
    x.en = (!kLean && a.entropy) ? a.entropy[j] : 0.f;
    x.ad = (!kLean && a.adv_per_token) ? a.adv[j] : 0.f;
    if (!ok) x = TokIn{0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    return x;
}

__device__ __forceinline__ void token_contrib_v(const meshy_ppo_args& a, const TokIn& x, float A, float w_doc,
                                                Contrib& c) {
    const float nw = x.nw;
    const float ol = x.ol;
    const float mk = x.mk;
    const float lr = nw - ol;
    const float ratio = expf(lr);
    const float u = ratio * A;
    const float cl = t_clamp(ratio, 1.f - a.clip_low, 1.f + a.clip_high) * A;
    float pg = -t_min(u, cl);
    float tis = ratio;
    bool tm = true;
    if (a.use_icepop) {
        tis = expf(ol - x.ro);
        tm = (tis >= a.tis_min) && (tis <= a.tis_max);
        const float weight = tm ? tis : 0.f;
        pg = (tm ? pg : 0.f) * weight;
    } else if (a.use_tis) {
        tm = (ratio >= a.tis_min) && (ratio <= a.tis_max);
        pg = tm ? pg : 0.f;
    }
    c.seg[0] = pg * mk;
    c.seg[1] = mk;
    c.seg[2] = ratio * mk;
    c.seg[3] = ratio * ratio * mk;
    c.seg[4] = (a.positive_lm_coef != 0.f) ? -nw * w_doc * mk : 0.f;
    c.tok[TS_TIS] = tis * mk;
    c.tok[TS_RATIO] = ratio * mk;
    c.tok[TS_CLIP] = ((ratio < 1.f - a.clip_low) || (ratio > 1.f + a.clip_high)) ? mk : 0.f * mk;
    c.tok[TS_TIS_MASKED] = tm ? 0.f * mk : mk;
    c.tok[TS_COUNT] = mk;
    c.tok[TS_KL] = -lr * mk;
    c.tok[TS_LR_ABS] = fabsf(lr) * mk;
    c.tok[TS_K3] = 0.f;
    c.tok[TS_LOGDIFF] = 0.f;
    if (a.rollout_lp) {
        const float train_lp = a.train_lp_is_old ? ol : nw;
        const float diff = x.ro - train_lp;
        const float lrt = t_clamp(diff, -10.f, 10.f);
        const float k3 = expf(lrt) - lrt - 1.f;
        c.tok[TS_K3] = nan_to_num(k3) * mk;
        c.tok[TS_LOGDIFF] = nan_to_num(fabsf(diff)) * mk;
    }
    c.tok[TS_ENT] = a.entropy ? x.en * mk : 0.f;
}

// d(total loss)/d new_lp of one token (gD = grad_loss * D_d).
__device__ __forceinline__ float token_grad_v(const meshy_ppo_args& a, const TokIn& x, float A, float w_doc,
                                              float gD) {
    const float lo_c = 1.f - a.clip_low;
    const float hi_c = 1.f + a.clip_high;
    const float nw = x.nw;
    const float ol = x.ol;
    const float mk = x.mk;
    const float ratio = expf(nw - ol);
    const float u = ratio * A;
    const float c = t_clamp(ratio, lo_c, hi_c) * A;
    // grad of pg_per_token (before masking) w.r.t. pg = -min(u, c)
    float g = gD * mk;
    if (a.use_icepop) {
        const float tis = expf(ol - x.ro);
        const bool tm = (tis >= a.tis_min) && (tis <= a.tis_max);
        g = tm ? g * tis : 0.f;
    } else if (a.use_tis) {
        const bool tm = (ratio >= a.tis_min) && (ratio <= a.tis_max);
        g = tm ? g : 0.f;
    }
    const float gm = -g;  // through the negation
    float gu, gc;
    if (u == c) {
        gu = 0.5f * gm;
        gc = 0.5f * gm;
    } else {
        gu = (u > c) ? 0.f : gm;
        gc = (u < c) ? 0.f : gm;
    }
    const float in_range = (ratio >= lo_c && ratio <= hi_c) ? 1.f : 0.f;
    const float g_ratio = gu * A + (gc * A) * in_range;
    float gn = g_ratio * ratio;
    if (a.positive_lm_coef != 0.f) gn += (gD * a.positive_lm_coef) * (-(w_doc * mk));
    return gn;
}

// The document of token i, clamped to the slots so that malformed ids stay in bounds.
__device__ __forceinline__ int64_t doc_at(const meshy_ppo_args& a, int64_t i) {
    return min(max(a.doc_ids[i], static_cast<int64_t>(0)), a.n_docs);
}

// The combine, run by the last tile workgroup once every tile's partials are
// visible: per-document totals in tile order and their loss / ESS terms, then
// every token-level sum, in one fixed-order block reduction (fp64 across
// threads).  seg_cnt_out receives each slot's masked token count.
template <int NT>
__device__ __forceinline__ void ppo_combine(const meshy_ppo_args& a, const Workspace& ws, float* __restrict__ out,
                                            float* __restrict__ seg_cnt_out) {
    __shared__ double s_red[NT / kWave][kFinalVals];
    __shared__ double s_tot[kFinalVals];
    const int64_t n_slots = a.n_docs + 1;
    const int64_t n_tiles = n_tiles_of(a.n_tokens);
    double v[kFinalVals];
#pragma unroll
    for (int k = 0; k < kFinalVals; ++k) v[k] = 0.0;
    // Token-level sums of every tile: v[4..13], four tiles per step with every
    // load of a step issued before any is added (indices clamped, extra tiles
    // dropped by a select).  Issued first: they do not wait on the offsets.
    constexpr int kStep = 4;
    for (int64_t b0 = threadIdx.x; b0 < n_tiles; b0 += NT * kStep) {
        float t[kStep][kTokSums];
#pragma unroll
        for (int u = 0; u < kStep; ++u) {
            const int64_t b = min(b0 + static_cast<int64_t>(u) * NT, n_tiles - 1);
#pragma unroll
            for (int k = 0; k < kTokSums; ++k) t[u][k] = ws.tok[b * kTokSums + k];
        }
#pragma unroll
        for (int u = 0; u < kStep; ++u) {
            const bool ok = b0 + static_cast<int64_t>(u) * NT < n_tiles;
#pragma unroll
            for (int k = 0; k < kTokSums; ++k) v[4 + k] += ok ? t[u][k] : 0.f;
        }
    }
    // Per-document totals (tile order) and their contributions: v[0..3] =
    // loss terms, positive-LM terms, ESS terms, documents with tokens.  The
    // first kDocTiles tiles of a document are loaded together (indices clamped
    // to its last tile, which is a written pair; an empty document's loads are
    // dropped), so a document of up to kDocTiles tiles costs one round trip
    // after its offsets.  Sums run in tile order either way.
    constexpr int kDocTiles = 4;
    for (int64_t d = threadIdx.x; d < n_slots; d += NT) {
        // Clamped to the tokens, so that malformed offsets stay in bounds.
        const int64_t lo = min(max(a.seg_offsets[d], static_cast<int64_t>(0)), a.n_tokens);
        const int64_t hi = min(max(a.seg_offsets[d + 1], lo), a.n_tokens);
        const int64_t b0 = lo / kTile;
        const int64_t b1 = max(hi - 1, static_cast<int64_t>(0)) / kTile;
        float t[kDocTiles][kSegSums];
#pragma unroll
        for (int u = 0; u < kDocTiles; ++u) {
            const float* src = ws.seg + (min(b0 + u, b1) + d) * kSegSums;
#pragma unroll
            for (int k = 0; k < kSegSums; ++k) t[u][k] = src[k];
        }
        float sg[kSegSums] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kDocTiles; ++u) {
            const bool ok = hi > lo && b0 + u <= b1;
#pragma unroll
            for (int k = 0; k < kSegSums; ++k) sg[k] += ok ? t[u][k] : 0.f;
        }
        if (hi > lo) {
            for (int64_t b = b0 + kDocTiles; b <= b1; ++b) {
                const float* src = ws.seg + (b + d) * kSegSums;
#pragma unroll
                for (int k = 0; k < kSegSums; ++k) sg[k] += src[k];
            }
        }
        if (seg_cnt_out) seg_cnt_out[d] = sg[1];
        if (d < a.n_docs) {
            if (a.per_token_loss) {
                v[0] += sg[0];
                v[1] += sg[4];
            } else {
                const float c = fmaxf(sg[1], 1.f);
                v[0] += sg[0] / c;
                v[1] += sg[4] / c;
            }
            if (sg[1] > 0.f) {
                v[2] += (sg[2] * sg[2]) / (fmaxf(sg[1], 1.f) * fmaxf(sg[3], 1e-8f));
                v[3] += 1.0;
            }
        }
    }
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
#pragma unroll
    for (int k = 0; k < kFinalVals; ++k) v[k] = wave_sum(v[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < kFinalVals; ++k) s_red[wid][k] = v[k];
    }
    __syncthreads();
    if (threadIdx.x < kFinalVals) {
        double s = 0.0;
        for (int w = 0; w < NT / kWave; ++w) s += s_red[w][threadIdx.x];
        s_tot[threadIdx.x] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const double* t = s_tot;
        const double den = a.per_token_loss ? static_cast<double>(max<int64_t>(1, a.n_tokens_global))
                                            : static_cast<double>(max<int64_t>(1, a.n_docs_global));
        const float loss = static_cast<float>(t[0] / den);
        const float pos = static_cast<float>(t[1] / den);
        const float cp = static_cast<float>(max(1, a.cp_degree));
        const double* tok = t + 4;
        out[MESHY_PPO_LOSS] = loss;
        out[MESHY_PPO_TOTAL_LOSS] = loss + a.positive_lm_coef * pos;
        out[MESHY_PPO_POSITIVE_LM_LOSS] = pos;
        out[MESHY_PPO_TIS_RATIO_SUM] = static_cast<float>(tok[TS_TIS]);
        out[MESHY_PPO_RATIO_SUM] = static_cast<float>(tok[TS_RATIO]);
        out[MESHY_PPO_CLIP_SUM] = static_cast<float>(tok[TS_CLIP]);
        out[MESHY_PPO_TIS_MASKED_SUM] = static_cast<float>(tok[TS_TIS_MASKED]);
        out[MESHY_PPO_TOKEN_COUNT] = static_cast<float>(tok[TS_COUNT]);
        out[MESHY_PPO_KL_SUM] = static_cast<float>(tok[TS_KL]);
        out[MESHY_PPO_LOG_RATIO_ABS_SUM] = static_cast<float>(tok[TS_LR_ABS]);
        out[MESHY_PPO_ESS_SUM] = static_cast<float>(t[2]) / cp;
        out[MESHY_PPO_DOC_COUNT] = static_cast<float>(t[3]) / cp;
        out[MESHY_PPO_TRAIN_ROLLOUT_KL_SUM] = static_cast<float>(tok[TS_K3]);
        out[MESHY_PPO_TRAIN_ROLLOUT_LOGDIFF_ABS_SUM] = static_cast<float>(tok[TS_LOGDIFF]);
        out[MESHY_PPO_ENTROPY_SUM] = static_cast<float>(tok[TS_ENT]);
    }
}

// kLean: the configuration without IcePop, rollout log-probs, entropy or
// per-token advantages, whose per-token registers are then not allocated.
template <bool kLean>
__global__ __launch_bounds__(kThreads) void k_ppo_tiles(meshy_ppo_args a, Workspace ws, bool vec) {
    __shared__ float s_red[kWaves][kTokSums + kFastDocs * kSegSums];
    const int64_t b = blockIdx.x;
    const int64_t t0 = b * kTile;
    const int64_t t1 = min(t0 + kTile, a.n_tokens);
    const int lane = threadIdx.x % kWave;
    const int wid = threadIdx.x / kWave;
    // The tile's tokens (thread t holds tokens 4t .. 4t+3 of each of the
    // tile's 1024-token halves: 16-byte loads when every array is aligned),
    // then its document range and the boundaries inside it.
    constexpr int kPer = static_cast<int>(kTile / kThreads);
    // The document range is loaded first: the per-document loads that depend
    // on it then issue while the token loads are still in flight.
    const int64_t d_first = doc_at(a, t0);
    const int64_t nd = max(doc_at(a, t1 - 1), d_first) - d_first + 1;
    TokIn in[kPer];
#pragma unroll
    for (int h = 0; h < kPer / 4; ++h) {
        const int64_t i4 = t0 + h * (4 * kThreads) + 4 * threadIdx.x;
        if (vec && i4 + 4 <= t1) {
            const float4 nw = *reinterpret_cast<const float4*>(a.new_lp + i4);
            const float4 ol = *reinterpret_cast<const float4*>(a.old_lp + i4);
            const float4 mk = *reinterpret_cast<const float4*>(a.mask + i4);
            float4 ro = make_float4(0.f, 0.f, 0.f, 0.f), en = ro, ad = ro;
            if (!kLean && a.rollout_lp) ro = *reinterpret_cast<const float4*>(a.rollout_lp + i4);
            if (!kLean && a.entropy) en = *reinterpret_cast<const float4*>(a.entropy + i4);
            if (!kLean && a.adv_per_token) ad = *reinterpret_cast<const float4*>(a.adv + i4);
            in[4 * h + 0] = TokIn{nw.x, ol.x, mk.x, ro.x, en.x, ad.x};
            in[4 * h + 1] = TokIn{nw.y, ol.y, mk.y, ro.y, en.y, ad.y};
            in[4 * h + 2] = TokIn{nw.z, ol.z, mk.z, ro.z, en.z, ad.z};
            in[4 * h + 3] = TokIn{nw.w, ol.w, mk.w, ro.w, en.w, ad.w};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) in[4 * h + e] = load_tok<kLean>(a, i4 + e, i4 + e < t1);
        }
    }
    // Unit gradient of each token (token mean: the loss's gradient is known
    // up to the scalar the backward multiplies in).
    float* const gu = (a.grad_unit && a.per_token_loss) ? a.grad_unit : nullptr;
    const float tok_scale = 1.f / static_cast<float>(max<int64_t>(1, a.n_tokens_global));
    float acc[kTokSums];
#pragma unroll
    for (int k = 0; k < kTokSums; ++k) acc[k] = 0.f;

    if (nd <= kFastDocs) {
        float A_d[kFastDocs], W_d[kFastDocs];
        int64_t bnd[kFastDocs];  // bnd[r]: first token of slot r (slots past nd: never reached)
#pragma unroll
        for (int r = 0; r < kFastDocs; ++r) {
            const int64_t d = d_first + r;
            const bool real = r < nd && d < a.n_docs;
            A_d[r] = (!a.adv_per_token && real) ? a.adv[d] : 0.f;
            W_d[r] = (a.positive_lm_weights && real) ? a.positive_lm_weights[d] : 0.f;
            bnd[r] = (r > 0 && r < nd) ? a.seg_offsets[d] : INT64_MAX;
        }
        // A thread's tokens (i = t0 + q * kThreads + tid) go through the tile's
        // documents in order, so the document sums accumulate in one run that
        // is flushed into its slot when the document changes (at most nd - 1
        // times).  Token sums that equal sums of the slots (mask count, ratio,
        // and the TIS ratio without IcePop) or that are zero with a feature off
        // are not accumulated per token.
        float sg[kFastDocs][kSegSums];
#pragma unroll
        for (int r = 0; r < kFastDocs; ++r)
#pragma unroll
            for (int k = 0; k < kSegSums; ++k) sg[r][k] = 0.f;
        float run[kSegSums] = {0.f, 0.f, 0.f, 0.f, 0.f};
        auto flush = [&](int slot) {
#pragma unroll
            for (int r = 0; r < kFastDocs; ++r)
#pragma unroll
                for (int k = 0; k < kSegSums; ++k) sg[r][k] += (slot == r) ? run[k] : 0.f;
#pragma unroll
            for (int k = 0; k < kSegSums; ++k) run[k] = 0.f;
        };
        const bool pos_lm = a.positive_lm_coef != 0.f;
        const float lo_c = 1.f - a.clip_low, hi_c = 1.f + a.clip_high;
        float gval[kPer];  // the unit gradient of the thread's tokens, stored after the loop
#pragma unroll
        for (int q = 0; q < kPer; ++q) gval[q] = 0.f;
        int cur = 0;
        float A = A_d[0], W = W_d[0];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int64_t i = t0 + (q / 4) * (4 * kThreads) + 4 * threadIdx.x + (q % 4);
            if (i >= t1) break;
            int slot = 0;
#pragma unroll
            for (int r = 1; r < kFastDocs; ++r) slot += (i >= bnd[r]) ? 1 : 0;
            if (slot != cur) {
                flush(cur);
                cur = slot;
#pragma unroll
                for (int r = 0; r < kFastDocs; ++r) {
                    A = (slot == r) ? A_d[r] : A;
                    W = (slot == r) ? W_d[r] : W;
                }
            }
            const TokIn& x = in[q];
            const float mk = x.mk;
            const float lr = x.nw - x.ol;
            const float ratio = expf(lr);
            const float At = (!kLean && a.adv_per_token) ? x.ad : A;
            float pg = -t_min(ratio * At, t_clamp(ratio, lo_c, hi_c) * At);
            bool tm = true;
            float tis = ratio;
            if (!kLean && a.use_icepop) {
                tis = expf(x.ol - x.ro);
                tm = (tis >= a.tis_min) && (tis <= a.tis_max);
                pg = (tm ? pg : 0.f) * (tm ? tis : 0.f);
            } else if (a.use_tis) {
                tm = (ratio >= a.tis_min) && (ratio <= a.tis_max);
                pg = tm ? pg : 0.f;
            }
            const float rm = ratio * mk;
            run[0] = fmaf(pg, mk, run[0]);
            run[1] += mk;
            run[2] += rm;
            run[3] = fmaf(ratio, rm, run[3]);
            if (pos_lm) run[4] = fmaf(-x.nw * W, mk, run[4]);
            acc[TS_CLIP] += ((ratio < lo_c) || (ratio > hi_c)) ? mk : 0.f * mk;
            acc[TS_KL] = fmaf(-lr, mk, acc[TS_KL]);
            acc[TS_LR_ABS] = fmaf(fabsf(lr), mk, acc[TS_LR_ABS]);
            if (!kLean && a.use_icepop) acc[TS_TIS] = fmaf(tis, mk, acc[TS_TIS]);
            if (a.use_icepop || a.use_tis) acc[TS_TIS_MASKED] += tm ? 0.f * mk : mk;
            if (!kLean && a.rollout_lp) {
                const float diff = x.ro - (a.train_lp_is_old ? x.ol : x.nw);
                const float lrt = t_clamp(diff, -10.f, 10.f);
                acc[TS_K3] = fmaf(nan_to_num(expf(lrt) - lrt - 1.f), mk, acc[TS_K3]);
                acc[TS_LOGDIFF] = fmaf(nan_to_num(fabsf(diff)), mk, acc[TS_LOGDIFF]);
            }
            if (!kLean && a.entropy) acc[TS_ENT] = fmaf(x.en, mk, acc[TS_ENT]);
            if (gu) {
                const bool real = d_first + slot < a.n_docs;  // the padding slot is not in the loss
                gval[q] = real ? token_grad_v(a, x, At, W, tok_scale) : 0.f;
            }
        }
        flush(cur);
        if (gu) {
            // Nontemporal: the backward reads the unit gradient once, from
            // HBM, and kept out of the L2 it does not slow the kernel's end
            // (21.4 against 23.5 us for the forward and backward of 1.83 M
            // tokens, A/B on one box).  One 16-byte store per thread and half:
            // the wave writes whole lines (a 4-byte store per token wrote
            // 16-byte-strided pieces that the counters saw as 3.8x the bytes).
#pragma unroll
            for (int h = 0; h < kPer / 4; ++h) {
                const int64_t i4 = t0 + h * (4 * kThreads) + 4 * threadIdx.x;
                if (vec && i4 + 4 <= t1) {
                    const f32x4 g4 = {gval[4 * h], gval[4 * h + 1], gval[4 * h + 2], gval[4 * h + 3]};
                    __builtin_nontemporal_store(g4, reinterpret_cast<f32x4*>(gu + i4));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (i4 + e < t1) __builtin_nontemporal_store(gval[4 * h + e], gu + i4 + e);
                }
            }
        }
        // The token sums that are sums of the slots.
#pragma unroll
        for (int r = 0; r < kFastDocs; ++r) {
            acc[TS_COUNT] += sg[r][1];
            acc[TS_RATIO] += sg[r][2];
        }
        if (!a.use_icepop) acc[TS_TIS] = acc[TS_RATIO];
        // One block reduction of the token sums and the nd x 5 document sums
        // (the sums that are zero with a feature off stay zero).
        const bool need[kTokSums] = {true, true, true, a.use_icepop || a.use_tis, true, true, true,
                                     a.rollout_lp != nullptr, a.rollout_lp != nullptr, a.entropy != nullptr};
#pragma unroll
        for (int k = 0; k < kTokSums; ++k)
            if (need[k]) acc[k] = wave_sum(acc[k]);
#pragma unroll
        for (int r = 0; r < kFastDocs; ++r) {
            if (r < nd) {
#pragma unroll
                for (int k = 0; k < kSegSums; ++k) sg[r][k] = wave_sum(sg[r][k]);
            }
        }
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < kTokSums; ++k) s_red[wid][k] = acc[k];
#pragma unroll
            for (int r = 0; r < kFastDocs; ++r)
#pragma unroll
                for (int k = 0; k < kSegSums; ++k) s_red[wid][kTokSums + r * kSegSums + k] = sg[r][k];
        }
        __syncthreads();
        // Every document between the first and the last lies within the tile
        // (or is empty, with zero sums), so its (tile, document) pair is its own.
        const int j = threadIdx.x;
        if (j < kTokSums + nd * kSegSums) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) v += s_red[w][j];
            if (j < kTokSums) {
                ws.tok[b * kTokSums + j] = v;
            } else {
                const int r = (j - kTokSums) / kSegSums;
                const int k = (j - kTokSums) % kSegSums;
                ws.seg[(b + d_first + r) * kSegSums + k] = v;
            }
        }
        return;
    }

    // Many documents in this tile: one wavefront per (tile, document) pair.
    for (int64_t d = d_first + wid; d < d_first + nd; d += kWaves) {
        const int64_t lo = max(a.seg_offsets[d], t0);
        const int64_t hi = min(a.seg_offsets[d + 1], t1);
        if (lo >= hi) continue;
        const bool real = d < a.n_docs;
        const float A_doc = (!a.adv_per_token && real) ? a.adv[d] : 0.f;
        const float w_doc = (a.positive_lm_weights && real) ? a.positive_lm_weights[d] : 0.f;
        float sg[kSegSums] = {0.f, 0.f, 0.f, 0.f, 0.f};
        for (int64_t i = lo + lane; i < hi; i += kWave) {
            Contrib c;
            const TokIn x = load_tok(a, i, true);
            const float At = a.adv_per_token ? x.ad : A_doc;
            token_contrib_v(a, x, At, w_doc, c);
#pragma unroll
            for (int k = 0; k < kSegSums; ++k) sg[k] += c.seg[k];
#pragma unroll
            for (int k = 0; k < kTokSums; ++k) acc[k] += c.tok[k];
            if (gu) __builtin_nontemporal_store(real ? token_grad_v(a, x, At, w_doc, tok_scale) : 0.f, gu + i);
        }
#pragma unroll
        for (int k = 0; k < kSegSums; ++k) sg[k] = wave_sum(sg[k]);
        if (lane == 0) {
            float* dst = ws.seg + (b + d) * kSegSums;
#pragma unroll
            for (int k = 0; k < kSegSums; ++k) dst[k] = sg[k];
        }
    }
#pragma unroll
    for (int k = 0; k < kTokSums; ++k) acc[k] = wave_sum(acc[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < kTokSums; ++k) s_red[wid][k] = acc[k];
    }
    __syncthreads();
    if (threadIdx.x < kTokSums) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += s_red[w][threadIdx.x];
        ws.tok[b * kTokSums + threadIdx.x] = v;
    }
}

constexpr int kBwdItems = 4;  // tokens per thread of k_ppo_bwd, strided by the workgroup (fastest of 2, 4, 8, 16)

// Three phases per thread: every token's inputs, then every token's document
// factors, then the arithmetic and the stores.  All loads take indices that are
// valid for every lane (token 0 past the end; the document clamped into the
// per-document arrays, whose value is dropped for the padding slot), so none
// sits behind a per-lane branch, which would wait for each load in turn.  The
// entropy is not read: the gradient does not depend on it.
__global__ __launch_bounds__(kThreads) void k_ppo_bwd(meshy_ppo_args a, const float* __restrict__ seg_cnt,
                                                      const float* __restrict__ grad_loss,
                                                      float* __restrict__ grad_new) {
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kThreads * kBwdItems + threadIdx.x;
    const float G = grad_loss[0];
    TokIn in[kBwdItems];
    int64_t d[kBwdItems];
#pragma unroll
    for (int q = 0; q < kBwdItems; ++q) {
        const int64_t i = t0 + q * kThreads;
        const int64_t j = i < a.n_tokens ? i : 0;
        in[q].nw = a.new_lp[j];
        in[q].ol = a.old_lp[j];
        in[q].mk = a.mask[j];
        in[q].ro = a.use_icepop ? a.rollout_lp[j] : 0.f;
        in[q].en = 0.f;
        in[q].ad = a.adv_per_token ? a.adv[j] : 0.f;
        d[q] = doc_at(a, j);
    }
    const bool have_docs = a.n_docs > 0;
    const int64_t last = have_docs ? a.n_docs - 1 : 0;
    float A[kBwdItems], W[kBwdItems], C[kBwdItems];
#pragma unroll
    for (int q = 0; q < kBwdItems; ++q) {
        const int64_t dc = min(d[q], last);
        A[q] = (have_docs && !a.adv_per_token) ? a.adv[dc] : 0.f;
        W[q] = (have_docs && a.positive_lm_weights) ? a.positive_lm_weights[dc] : 0.f;
        C[q] = (have_docs && !a.per_token_loss) ? seg_cnt[dc] : 0.f;
    }
    const float tok_scale = 1.f / static_cast<float>(max<int64_t>(1, a.n_tokens_global));
    const float docs_g = static_cast<float>(max<int64_t>(1, a.n_docs_global));
#pragma unroll
    for (int q = 0; q < kBwdItems; ++q) {
        const int64_t i = t0 + q * kThreads;
        const bool real = d[q] < a.n_docs;  // the padding slot is not in the loss
        const float Aq = a.adv_per_token ? in[q].ad : (real ? A[q] : 0.f);
        const float Wq = real ? W[q] : 0.f;
        const float scale = !real ? 0.f : (a.per_token_loss ? tok_scale : 1.f / (fmaxf(C[q], 1.f) * docs_g));
        const float g = token_grad_v(a, in[q], Aq, Wq, G * scale);
        if (i < a.n_tokens) grad_new[i] = g;
    }
}

// 256 threads: as fast as 1024 here (the combine is bound by its chains of
// dependent loads), with a smaller register file to allocate.
constexpr int kCombineThreads = 256;

// One workgroup: the combine of every tile's partials.
__global__ __launch_bounds__(kCombineThreads) void k_ppo_combine(meshy_ppo_args a, Workspace ws,
                                                                 float* __restrict__ out,
                                                                 float* __restrict__ seg_cnt_out) {
    ppo_combine<kCombineThreads>(a, ws, out, seg_cnt_out);
}

// Token mean: grad_new = grad_loss * unit gradient, 4 tokens per thread
// (16-byte accesses when both buffers are aligned).
__global__ __launch_bounds__(kThreads) void k_ppo_scale(const float* __restrict__ gu,
                                                        const float* __restrict__ grad_loss,
                                                        float* __restrict__ grad_new, int64_t n, bool vec) {
    const float G = grad_loss[0];
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 4;
    if (vec && i + 4 <= n) {
        float4 v = *reinterpret_cast<const float4*>(gu + i);
        v.x *= G;
        v.y *= G;
        v.z *= G;
        v.w *= G;
        *reinterpret_cast<float4*>(grad_new + i) = v;
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (i + k < n) grad_new[i + k] = G * gu[i + k];
}

// seg_offsets[d] = first token with id >= d, for sorted ids: token i writes
// every d in (ids[i-1], ids[i]]; the slots after the last id get n.
typedef long long i64x2 __attribute__((ext_vector_type(2)));
constexpr int kSegItems = 8;  // doc ids per thread of k_segment_offsets

// Thread t owns the boundaries before positions i0 .. i0 + 7 (i0 = 8 t) and,
// for the last thread, the one at n: every document slot whose first token is
// there (empty slots included) gets offset i.  16-byte loads when aligned.
__global__ __launch_bounds__(kThreads) void k_segment_offsets(const int64_t* __restrict__ ids, int64_t n,
                                                              int64_t n_slots, bool vec, int64_t* __restrict__ off,
                                                              int32_t* __restrict__ unsorted) {
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kSegItems;
    if (i0 > n) return;
    int64_t v[kSegItems + 1];  // v[0] = ids[i0 - 1], v[k + 1] = ids[i0 + k] (n_slots from n on)
    v[0] = (i0 == 0) ? -1 : ids[i0 - 1];
    if (vec && i0 + kSegItems <= n) {
#pragma unroll
        for (int q = 0; q < kSegItems / 2; ++q) {
            const i64x2 w = *reinterpret_cast<const i64x2*>(ids + i0 + 2 * q);
            v[2 * q + 1] = w.x;
            v[2 * q + 2] = w.y;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kSegItems; ++k) v[k + 1] = (i0 + k < n) ? ids[i0 + k] : n_slots;
    }
#pragma unroll
    for (int k = 0; k < kSegItems; ++k) {
        const int64_t i = i0 + k;
        if (i > n) break;
        const int64_t prev = v[k];
        const int64_t cur = v[k + 1];
        if (unsorted && i < n) {
            // Rare error paths: an atomic keeps both reasons when both occur.
            if (i > 0 && prev > cur) atomicOr(unsorted, 1);
            if (cur < 0 || cur >= n_slots) atomicOr(unsorted, 2);
        }
        const int64_t lo = max<int64_t>(prev + 1, 0);
        const int64_t hi = min<int64_t>(cur, n_slots - 1);
        for (int64_t d = lo; d <= hi; ++d) off[d] = i;
    }
    if (i0 == 0) off[n_slots] = n;
}

int validate(const meshy_ppo_args& a, const char* who) {
    if (a.n_tokens < 0 || a.n_docs < 0) return set_error(MESHY_EINVAL, "%s: negative sizes", who);
    // Without tokens the per-token arrays may be NULL (an empty tensor has no
    // storage); the document slots still get their sums.
    const bool tok = a.n_tokens > 0;
    if ((tok && (!a.new_lp || !a.old_lp || !a.mask || !a.doc_ids)) || !a.seg_offsets ||
        (a.n_docs > 0 && !a.adv && !a.adv_per_token) || (tok && a.adv_per_token && !a.adv))
        return set_error(MESHY_ENULL, "%s: new_lp, old_lp, mask, adv, seg_offsets and doc_ids are required", who);
    if (a.use_icepop && !a.rollout_lp) return set_error(MESHY_EINVAL, "%s: IcePop requires rollout log-probabilities", who);
    if (a.positive_lm_coef != 0.f && !a.positive_lm_weights && a.n_docs > 0)
        return set_error(MESHY_EINVAL, "%s: Positive LM loss requires group weights", who);
    if (a.n_tokens > INT32_MAX) return set_error(MESHY_EINVAL, "%s: too many tokens", who);
    if (a.n_docs >= INT32_MAX) return set_error(MESHY_EINVAL, "%s: too many documents", who);
    return MESHY_OK;
}

}  // namespace
}  // namespace meshy

extern "C" size_t meshy_ppo_workspace_size(int64_t n_tokens, int64_t n_docs) {
    if (n_tokens < 0 || n_docs < 0) return 0;
    return meshy::ws_bytes(n_tokens, n_docs);
}

extern "C" int meshy_ppo_loss_fwd(const meshy_ppo_args* args, float* out, float* seg_cnt, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (!args || !out) return set_error(MESHY_ENULL, "meshy_ppo_loss_fwd: args and out are required");
    const meshy_ppo_args& a = *args;
    int rc = validate(a, "meshy_ppo_loss_fwd");
    if (rc) return rc;
    if (!a.workspace || a.workspace_bytes < ws_bytes(a.n_tokens, a.n_docs))
        return set_error(MESHY_ESPACE, "meshy_ppo_loss_fwd: workspace needs %zu bytes",
                         ws_bytes(a.n_tokens, a.n_docs));
    const Workspace ws = ws_of(a.workspace, a.n_tokens);
    const int64_t nt = n_tiles_of(a.n_tokens);
    if (nt == 0) {
        hipLaunchKernelGGL(k_ppo_combine, dim3(1), dim3(kCombineThreads), 0, stream, a, ws, out, seg_cnt);
        return check_launch("meshy_ppo_loss_fwd(combine)");
    }
    const bool lean = !a.use_icepop && !a.rollout_lp && !a.entropy && !a.adv_per_token;
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool vec = al16(a.new_lp) && al16(a.old_lp) && al16(a.mask) && al16(a.rollout_lp) && al16(a.entropy) &&
                     (!a.adv_per_token || al16(a.adv)) && al16(a.grad_unit);
    if (lean)
        hipLaunchKernelGGL(k_ppo_tiles<true>, dim3(static_cast<unsigned>(nt)), dim3(kThreads), 0, stream, a, ws, vec);
    else
        hipLaunchKernelGGL(k_ppo_tiles<false>, dim3(static_cast<unsigned>(nt)), dim3(kThreads), 0, stream, a, ws, vec);
    rc = check_launch("meshy_ppo_loss_fwd(tiles)");
    if (rc) return rc;
    hipLaunchKernelGGL(k_ppo_combine, dim3(1), dim3(kCombineThreads), 0, stream, a, ws, out, seg_cnt);
    return check_launch("meshy_ppo_loss_fwd(combine)");
}

extern "C" int meshy_ppo_loss_bwd(const meshy_ppo_args* args, const float* seg_cnt, const float* grad_loss,
                                  float* grad_new, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (!args || !grad_loss)
        return set_error(MESHY_ENULL, "meshy_ppo_loss_bwd: args, grad_loss and grad_new are required");
    const meshy_ppo_args& a = *args;
    int rc = validate(a, "meshy_ppo_loss_bwd");
    if (rc) return rc;
    if (a.n_tokens == 0) return MESHY_OK;
    if (!grad_new) return set_error(MESHY_ENULL, "meshy_ppo_loss_bwd: args, grad_loss and grad_new are required");
    if (a.grad_unit && a.per_token_loss) {
        const int64_t nb = ceil_div(ceil_div(a.n_tokens, 4), static_cast<int64_t>(kThreads));
        const bool vec = reinterpret_cast<uintptr_t>(a.grad_unit) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(grad_new) % 16 == 0;
        hipLaunchKernelGGL(k_ppo_scale, dim3(static_cast<unsigned>(nb)), dim3(kThreads), 0, stream, a.grad_unit,
                           grad_loss, grad_new, a.n_tokens, vec);
        return check_launch("meshy_ppo_loss_bwd(scale)");
    }
    if (!seg_cnt) return set_error(MESHY_ENULL, "meshy_ppo_loss_bwd: seg_cnt is required without grad_unit");
    const int64_t nb = ceil_div(a.n_tokens, static_cast<int64_t>(kThreads) * kBwdItems);
    hipLaunchKernelGGL(k_ppo_bwd, dim3(static_cast<unsigned>(nb)), dim3(kThreads), 0, stream, a, seg_cnt,
                       grad_loss, grad_new);
    return check_launch("meshy_ppo_loss_bwd");
}

extern "C" int meshy_segment_offsets(const int64_t* doc_ids, int64_t n_tokens, int64_t n_slots,
                                     int64_t* seg_offsets, int32_t* unsorted, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (n_tokens < 0 || n_slots < 1) return set_error(MESHY_EINVAL, "meshy_segment_offsets: bad sizes");
    if (!seg_offsets || (n_tokens > 0 && !doc_ids))
        return set_error(MESHY_ENULL, "meshy_segment_offsets: NULL pointer");
    // n / 8 + 1 threads: the last one also owns the boundary at n.
    const int64_t blocks = ceil_div(n_tokens / kSegItems + 1, kThreads);
    if (blocks > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_segment_offsets: too many tokens");
    const bool vec = reinterpret_cast<uintptr_t>(doc_ids) % 16 == 0;
    hipLaunchKernelGGL(k_segment_offsets, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream,
                       doc_ids, n_tokens, n_slots, vec, seg_offsets, unsorted);
    return check_launch("meshy_segment_offsets");
}
