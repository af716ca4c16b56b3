/*
 * meshy_amd.h -- C ABI of libmeshy_amd.so, the MI355X (gfx950) implementation
 * of Meshy's ragged-batch path between rollout and trainer.
 *
 * Every entry point takes plain pointers and sizes.  Device pointers are HIP
 * device addresses; every device entry point is asynchronous on the stream it
 * is given and allocates nothing: scratch space comes in through a caller-owned
 * workspace whose size the matching *_workspace_size call reports.
 *
 * Return convention (all entry points):
 *     0   success
 *    <0   invalid argument (a MESHY_E* code); meshy_last_error() has the text
 *    >0   a hipError_t raised by a launch; meshy_last_error() has the text
 *
 * Reference paths below are relative to the OpenBMB/Meshy source tree.
 */
#ifndef MESHY_AMD_H
#define MESHY_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MESHY_OK 0
#define MESHY_EINVAL (-1)     /* bad argument value or shape            */
#define MESHY_ENULL (-2)      /* required pointer was NULL              */
#define MESHY_EALIGN (-3)     /* pointer or stride misaligned           */
#define MESHY_ESPACE (-4)     /* workspace too small                    */
#define MESHY_ENOTDIV (-5)    /* batch size not divisible by DP size    */
#define MESHY_EEMPTY (-6)     /* empty batch                            */

/* Text of the last error raised on the calling thread ("" when none). */
const char* meshy_last_error(void);
/* ABI version: bumped on any signature change. */
int meshy_abi_version(void);
/* An asynchronous host-to-device copy on `stream` (hipMemcpyAsync): the
 * staging buffers' transfers, issued without a framework tensor per copy.
 * From pinned memory it returns once queued; the caller keeps `src` intact
 * until the copy has run.  No counterpart in the reference, which copies
 * with torch's .to(device) (trainer.py:644-667, batch.py:126-178). */
int meshy_copy_to_device(void* dst, const void* src, size_t bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Token-budget planner (host).
 * Replaces build_plan (meshy/backend/titan/plan.py:211-288), including
 * _snake (plan.py:145-155), _pack_micros (plan.py:158-203) and filler_micro
 * (plan.py:206-208).  PlannerConfig's own validation (plan.py:60-81) stays
 * in the Python dataclass; this call re-checks what it relies on.
 * ---------------------------------------------------------------------- */
#define MESHY_LAYOUT_PADDED 0
#define MESHY_LAYOUT_PACKED 1

typedef struct meshy_planner_cfg {
    int32_t layout;               /* MESHY_LAYOUT_*                          */
    int32_t reserved;
    int64_t mini_batch_size;
    int64_t seq_len;
    int64_t align;
    int64_t max_tokens_per_micro; /* <= 0 means None                         */
    int64_t micro_batch_size;     /* <= 0 means None                         */
} meshy_planner_cfg;

/*
 * Caller-allocated plan tables.  With n samples, dp ranks,
 * n_local = n / dp and n_mini = ceil(n_local / mini_batch_size):
 *   local_indices        [dp * n_local]       Plan.local_indices
 *   mini_n_micro         [n_mini]             micros per mini (equal on all ranks)
 *   mini_n_docs_global   [n_mini]             MiniPlan.n_docs_global
 *   mini_n_tokens_global [n_mini]             MiniPlan.n_tokens_global
 *   mini_tokens_per_rank [n_mini * dp]        MiniPlan.tokens_per_rank
 *   micro_seq_len        [dp * n_local]       MicroPlan.seq_len, rank-major
 *   micro_doc_start      [dp * (n_local + 1)] CSR row pointer of each rank's micros
 *   doc_sample           [dp * n_local]       MicroPlan.sample_idx, flattened
 *   doc_len              [dp * n_local]       MicroPlan.doc_lens, flattened
 * Rank r's k-th micro (minis in order, fillers last within a mini) is
 * micro_seq_len[r*n_local + k] with documents
 * doc_*[r*n_local + micro_doc_start[r*(n_local+1) + k] ...
 *        r*n_local + micro_doc_start[r*(n_local+1) + k + 1]).
 * n_micro_total receives the micro count per rank (<= n_local).
 */
typedef struct meshy_plan_out {
    int32_t* local_indices;
    int32_t* mini_n_micro;
    int64_t* mini_n_docs_global;
    int64_t* mini_n_tokens_global;
    int64_t* mini_tokens_per_rank;
    int64_t* micro_seq_len;
    int32_t* micro_doc_start;
    int32_t* doc_sample;
    int64_t* doc_len;
    int32_t n_micro_total;
    int32_t reserved;
} meshy_plan_out;

int meshy_plan_build(const int64_t* lengths, const int64_t* loss_tokens, int64_t n,
                     int64_t dp_size, const meshy_planner_cfg* cfg, meshy_plan_out* out);

/* Concatenation of host byte ranges (host).
 * Replaces the per-sample torch.cat that stages jagged sample columns before
 * their host-to-device copy: the critic path's concatenation of masks and
 * values (meshy/backend/titan/trainer.py:644-667) and the per-sample slicing of
 * build_micro_batch (meshy/backend/titan/batch.py:126-178).  Piece i
 * (nbytes[i] bytes at srcs[i]) lands right after piece i - 1 in dst.  Runs on
 * up to max_threads threads of a persistent pool (<= 0: the pool's size, at
 * most 16), split by bytes; small gathers run on the calling thread. */
int meshy_host_gather(const void* const* srcs, const int64_t* nbytes, int64_t n, void* dst,
                      int max_threads);

/* The same concatenation of fp32 mask pieces into bytes (host): piece i
 * (counts[i] floats at srcs[i]) lands as counts[i] bytes right after piece
 * i - 1 in dst, each byte the float's value.  *binary is set to 1 when every
 * float was exactly +0.0 or 1.0 (bytes and floats then hold the same mask),
 * else to 0 (dst then holds no mask: stage the floats instead).  For masks
 * that are 0/1, as the reference's mask_assistant columns are, this quarters
 * the bytes the critic path copies to the device (trainer.py:644-667). */
int meshy_host_gather_mask_u8(const float* const* srcs, const int64_t* counts, int64_t n, uint8_t* dst,
                              int max_threads, int32_t* binary);
/* The same for int64 columns narrowed to int32 (host): counts[i] int64s of
 * srcs[i] land in dst as int32, and *fits is set to 1 when every value fits
 * in int32, else to 0 (dst then is not the column: stage the int64s).  The
 * OPD Teacher's top-k ids are vocabulary indices (opd.py:58-89), so this
 * halves the bytes their staging copies to the device. */
int meshy_host_gather_i32(const int64_t* const* srcs, const int64_t* counts, int64_t n, int32_t* dst,
                          int max_threads, int32_t* fits);

/* Per-sample planner inputs from a flat host mask (host).
 * Replaces TitanTrainer._sample_lengths (meshy/backend/titan/trainer.py:577-588):
 * sample i covers mask[offsets[i] .. offsets[i+1]); lengths[i] is its token
 * count and loss_tokens[i] = #(mask[1:L] > 0) with L = min(length, seq_len),
 * 0 when L <= 1. */
int meshy_sample_loss_tokens(const float* mask, const int64_t* offsets, int64_t n,
                             int64_t seq_len, int64_t* lengths, int64_t* loss_tokens);
/* The same over a mask staged as bytes (meshy_host_gather_mask_u8): a
 * nonzero byte counts. */
int meshy_sample_loss_tokens_u8(const uint8_t* mask, const int64_t* offsets, int64_t n,
                                int64_t seq_len, int64_t* lengths, int64_t* loss_tokens);

/* The host plan of one packing step in one call (host): what
 * TitanTrainer.plan_batch does before it builds each micro
 * (meshy/backend/titan/trainer.py:577-588, then plan.py:211-288):
 * meshy_sample_loss_tokens over the flat mask (cfg.seq_len), meshy_plan_build
 * into `plan`, then, for `rank`, the tables meshy_pack_micro_batches reads,
 * written where the caller stages them:
 *   micro_seq_len[k]     the rank's k-th micro's seq_len        [n_local]
 *   micro_out_off[k]     its first output element (seq_len x rows, rows = 1
 *                        packed, max(documents, 1) padded)    [n_local + 1]
 *   micro_doc_start[k]   its first document                   [n_local + 1]
 *   doc_sample[j]        document j's global sample index     [n_local]
 *   doc_len[j]           document j's length                  [n_local]
 * and the counts n_micro, n_docs, max_micro_elems, max_docs_per_micro.  The
 * errors are those of the two calls it makes. */
typedef struct meshy_step_plan_args {
    const void* mask;              /* [offsets[n]] host, fp32 (or bytes with
                                      mask_u8)                                */
    const int64_t* offsets;        /* [n + 1]                                 */
    int64_t n;
    int64_t dp_size;
    int64_t rank;
    meshy_planner_cfg cfg;
    meshy_plan_out plan;
    int64_t* lengths;              /* [n] out: tokens per sample              */
    int64_t* loss_tokens;          /* [n] out                                 */
    int64_t* micro_seq_len;        /* the rank's pack tables, out             */
    int64_t* micro_out_off;
    int32_t* micro_doc_start;
    int32_t* doc_sample;
    int64_t* doc_len;
    int64_t n_micro;               /* out                                     */
    int64_t n_docs;                /* out                                     */
    int64_t max_micro_elems;       /* out                                     */
    int64_t max_docs_per_micro;    /* out                                     */
    int32_t mask_u8;               /* 1: mask holds one byte per token        */
    int32_t reserved;
} meshy_step_plan_args;
int meshy_step_plan(meshy_step_plan_args* args);

/* ------------------------------------------------------------------------
 * Micro-batch materialisation (device).
 * Replaces build_micro_batch (meshy/backend/titan/batch.py:96-230): per-doc
 * shift-by-one (batch.py:91-93), doc_ids with the padding slot, per-doc
 * positions, cu_seqlens (batch.py:154-178, make_varlen_metadata 233-243).
 * One launch materialises any number of micros of one rank.
 * ---------------------------------------------------------------------- */
typedef struct meshy_pack_args {
    /* rank-local samples, concatenated (device) */
    const void* tokens;            /* [total] int32 or int64                  */
    int32_t tokens_elem_bytes;     /* 4 or 8                                  */
    int32_t layout;                /* MESHY_LAYOUT_*                          */
    const void* mask;              /* [total] mask_assistant, fp32 (or one
                                      byte per token, 0 or 1, with mask_u8)  */
    const float* logprobs;         /* [total] rollout logprobs, nullable      */
    const float* adv_tokens;       /* [total] per-token advantages (already on
                                      the next-token grid), nullable         */
    const float* adv_samples;      /* [n_samples] per-sample advantage
                                      (sample["advantage"]), nullable        */
    const int64_t* sample_offsets; /* [n_samples + 1]                         */
    int64_t n_samples;
    /* the micros to build (device) */
    int64_t n_micro;
    const int64_t* micro_seq_len;  /* [n_micro]                               */
    const int64_t* micro_out_off;  /* [n_micro + 1] element offset of each
                                      micro in the flat outputs (rows*seq_len
                                      elements per micro)                    */
    const int32_t* micro_doc_start;/* [n_micro + 1]                           */
    const int32_t* doc_sample;     /* [n_docs_total] rank-local sample index  */
    const int64_t* doc_len;        /* [n_docs_total] tokens entering forward  */
    int64_t max_micro_elems;       /* max over micros of rows*seq_len         */
    int64_t max_docs_per_micro;    /* max over micros of n_docs               */
    /* flat outputs (device) */
    int64_t* input_ids;
    int64_t* labels;
    int32_t* positions;
    float* mask_out;
    int64_t* doc_ids;
    float* rollout_lp;             /* nullable (need_rollout_lp=False)        */
    float* adv_tok;                /* nullable.  With adv_tokens: the sample's
                                      per-token advantages, unshifted
                                      (batch.py:166-170).  Otherwise, with
                                      adv_samples: the per-document advantage
                                      broadcast over the micro, 0 on the
                                      padding slot (trainer.py:753-756)      */
    float* adv_doc;                /* [n_docs_total] per-document advantage
                                      (batch.py:110-116), nullable; needs
                                      adv_samples                            */
    int32_t* doc_len_out;          /* [n_docs_total] Batch.lengths, nullable  */
    int32_t* cu_seqlens;           /* packed only, required there: micro k
                                      writes n_docs_k + 1 (+1 with a pad doc)
                                      values at micro_doc_start[k] + 2*k     */
    /* Optional Teacher Top-K columns of on-policy distillation (replaces
       layout_teacher_topk, meshy/backend/titan/opd.py:58-89): rows indexed
       by logits position, NOT shifted; zero outside the documents.  Off
       when teacher_k == 0. */
    int64_t teacher_k;
    const void* teacher_ids;       /* [total, teacher_k], int32 or int64      */
    const float* teacher_lps;      /* [total, teacher_k]                      */
    int64_t* teacher_ids_out;      /* [n_out, teacher_k]                      */
    float* teacher_lps_out;        /* [n_out, teacher_k]                      */
    int32_t teacher_ids_elem_bytes; /* 4 or 8 (0 reads as 4)                  */
    int32_t mask_u8;               /* 1: mask holds bytes (see mask)          */
    /* Optional int64 token offsets of each micro's n_docs + 1 document slots
       (padding slot last) over its flattened [rows, S] grid, the loss kernels'
       seg_offsets: micro k writes n_docs_k + 2 values at
       micro_doc_start[k] + 2*k.  Nullable. */
    int64_t* seg_offsets;
} meshy_pack_args;

int meshy_pack_micro_batches(const meshy_pack_args* args, hipStream_t stream);

/* ------------------------------------------------------------------------
 * GRPO group-normalised advantages (device).
 * Replaces grpo_advantage (meshy/worker/rollout.py:88-97) for all groups of a
 * batch at once: a size-1 group keeps its reward, otherwise
 * (r - mean) / clamp(unbiased std, min=1e-8).  Group g is rewards
 * [group_offsets[g], group_offsets[g+1]), clamped to [0, n_rewards).
 * ---------------------------------------------------------------------- */
int meshy_grpo_advantage(const float* rewards, int64_t n_rewards, const int64_t* group_offsets,
                         int64_t n_groups, float* advantages, hipStream_t stream);
/* The same over host arrays, for rewards the rollout worker holds on the host
 * (its per-group advantage plugin, rollout.py:580-587): no device round trip.
 * fp32 results, the mean and the variance summed in fp64. */
int meshy_grpo_advantage_host(const float* rewards, int64_t n_rewards, const int64_t* group_offsets,
                              int64_t n_groups, float* advantages);

/* ------------------------------------------------------------------------
 * Zero-variance group filter (device).
 * Replaces is_zero_variance_group (meshy/worker/rollout.py:100-115) for all
 * groups of a batch at once.  raw_rewards are the per-sample raw rewards in
 * float64 (the reference compares Python floats): sample.raw_reward when set,
 * else sample.reward.  flags[g] = 1 when max(raw) - min(raw) <= tolerance
 * with Python's max()/min() over group g (a NaN first element makes the
 * group 0, later NaNs are skipped), 1 for an empty group, else 0.  Group g is
 * raw_rewards[group_offsets[g], group_offsets[g+1]), clamped to
 * [0, n_rewards).  raw_rewards may be NULL when n_rewards is 0.
 * ---------------------------------------------------------------------- */
int meshy_zero_variance_groups(const double* raw_rewards, int64_t n_rewards, const int64_t* group_offsets,
                               int64_t n_groups, double tolerance, uint8_t* flags, hipStream_t stream);
/* The same filter over host arrays (raw_rewards, group_offsets and flags in
 * host memory), for rewards that are still on the host as the rollout worker
 * holds them (rollout.py:580-587): the same flags, no device round trip. */
int meshy_zero_variance_groups_host(const double* raw_rewards, int64_t n_rewards, const int64_t* group_offsets,
                                    int64_t n_groups, double tolerance, uint8_t* flags);

/* ------------------------------------------------------------------------
 * Fused packed log_softmax + gather + entropy (device), bf16 logits.
 * Replaces the chunk loop of TitanTrainer._forward_logprobs
 * (meshy/backend/titan/trainer.py:451-527) with its bodies _chunk_logprobs
 * (trainer.py:414-428: -cross_entropy(logits.float(), labels)) and
 * _chunk_entropy (trainer.py:430-449: logsumexp - sum softmax * z).
 *
 * logits element (b, t, v) lives at logits[b*stride_b + t*stride_t + v]
 * (strides in elements; stride_b, stride_t multiples of 8 and logits 16-byte
 * aligned take the vector path, anything else the unaligned path).
 * labels is contiguous [rows * T]; a label of -100 (cross_entropy's default
 * ignore_index) gives logp = 0; a label outside [0, V) gives NaN.
 * Outputs are contiguous [rows * T] fp32; each may be NULL.  lse is what the
 * backward consumes.
 * ---------------------------------------------------------------------- */
int meshy_logprob_entropy_fwd(const uint16_t* logits, int64_t rows, int64_t T, int64_t V,
                              int64_t stride_b, int64_t stride_t, const int64_t* labels,
                              float* logp, float* entropy, float* lse, hipStream_t stream);

/*
 * Backward of logp with respect to the logits:
 *   grad_logits[r, v] = grad_logp[r] * (onehot(label_r)[v] - exp(z[r, v] - lse[r]))
 * written as bf16 into a contiguous [rows * T, V] buffer.  Ignored labels
 * (-100) give a zero row, labels outside [0, V) a NaN row.  This is the
 * gradient torch autograd produces for the reference's checkpointed
 * -cross_entropy chunk (trainer.py:504-517).  The workspace holds two floats
 * per row (meshy_logprob_bwd_workspace_size(rows * T) bytes).
 */
size_t meshy_logprob_bwd_workspace_size(int64_t n_rows);
int meshy_logprob_bwd(const uint16_t* logits, int64_t rows, int64_t T, int64_t V,
                      int64_t stride_b, int64_t stride_t, const int64_t* labels,
                      const float* lse, const float* grad_logp, uint16_t* grad_logits,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Allocation-free variant of meshy_logprob_bwd.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory or pass a
 * workspace (code under HIP graph capture, tight training or serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * meshy_logprob_bwd; its two floats per row live in a static device array of
 * MESHY_NOALLOC_MAX_ROWS rows (2 MiB, one copy per GPU, held until the
 * process ends).  rows * T above that limit returns MESHY_ESPACE.  The call
 * allocates and frees nothing.  Calls that overlap on one GPU (on different
 * streams) share that array and race; calls on one stream are ordered.
 */
#define MESHY_NOALLOC_MAX_ROWS 262144
int meshy_logprob_bwd_noalloc(const uint16_t* logits, int64_t rows, int64_t T, int64_t V,
                              int64_t stride_b, int64_t stride_t, const int64_t* labels,
                              const float* lse, const float* grad_logp, uint16_t* grad_logits,
                              hipStream_t stream);

/* ------------------------------------------------------------------------
 * log_softmax(logits).gather(ids) over bf16 logits, and its backward (device).
 * Replaces gather_logprobs (meshy/backend/titan/topk_loss.py:40-57) and its
 * chunk body _chunk_gather_logprobs (topk_loss.py:35-37), with the
 * checkpointed recompute of the chunk in backward.
 *
 * ids is contiguous [rows * T, n_ids] int64 (1 <= n_ids <= 256); out the
 * same shape in fp32: out[r, k] = z[r, ids[r, k]] - lse[r].  An id of -100
 * gives 0, an id outside [0, V) NaN.  lse ([rows * T], nullable) receives
 * the per-row log-sum-exp the backward consumes.  Same logits layout rules
 * as meshy_logprob_entropy_fwd.
 *
 * Backward: grad_logits[r, v] = sum_k grad_out[r, k] onehot(ids[r, k])[v]
 *                               - (sum_k grad_out[r, k]) exp(z[r, v] - lse[r]),
 * ids of -100 contributing nothing, as bf16 into a contiguous [rows * T, V]
 * buffer; workspace as meshy_logprob_bwd.
 * ---------------------------------------------------------------------- */
int meshy_gather_logprobs_fwd(const uint16_t* logits, int64_t rows, int64_t T, int64_t V,
                              int64_t stride_b, int64_t stride_t, const int64_t* ids,
                              int64_t n_ids, float* out, float* lse, hipStream_t stream);
int meshy_gather_logprobs_bwd(const uint16_t* logits, int64_t rows, int64_t T, int64_t V,
                              int64_t stride_b, int64_t stride_t, const int64_t* ids,
                              int64_t n_ids, const float* lse, const float* grad_out,
                              uint16_t* grad_logits, void* workspace, size_t workspace_bytes,
                              hipStream_t stream);

/* ------------------------------------------------------------------------
 * Teacher Top-K with log-probabilities (device), bf16 logits.
 * Replaces teacher_topk (meshy/backend/titan/topk_loss.py:20-32):
 *   ids[r, :]      the k columns of the k largest logits of row r, by value
 *                  descending, equal values by ascending column;
 *   logprobs[r, :] those logits minus the row's logsumexp (fp32);
 *   lse[r]         the row's logsumexp (nullable).
 * Outputs are contiguous [rows * T, k]; 1 <= k <= min(64, V).  Same logits
 * layout rules as meshy_logprob_entropy_fwd.  NaN logits are never selected.
 * ---------------------------------------------------------------------- */
int meshy_topk_logprobs(const uint16_t* logits, int64_t rows, int64_t T, int64_t V,
                        int64_t stride_b, int64_t stride_t, int64_t k, int64_t* ids,
                        float* logprobs, float* lse, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Student Top-K distillation loss with its sums (device).
 * Replaces StudentTopKTrainer._distill_loss after the gather
 * (meshy/backend/titan/opd.py:164-197) and forward_kl_topk
 * (meshy/backend/titan/topk_loss.py:60-80).  Documents are contiguous token
 * ranges given by seg_offsets, as for the PPO loss.
 * ---------------------------------------------------------------------- */
enum meshy_distill_out {
    MESHY_DISTILL_LOSS = 0,                     /* opd.py:178-181          */
    MESHY_DISTILL_TOKEN_COUNT,
    MESHY_DISTILL_STUDENT_MASS_SUM,
    MESHY_DISTILL_TEACHER_MASS_SUM,
    MESHY_DISTILL_TRAIN_ROLLOUT_KL_SUM,          /* with rollout_lp only    */
    MESHY_DISTILL_TRAIN_ROLLOUT_LOGDIFF_ABS_SUM, /* with rollout_lp only    */
    MESHY_DISTILL_NOUT
};

typedef struct meshy_distill_args {
    const float* student;          /* [n_tokens, k + 1]: log-probs of the k
                                      Teacher ids then of the sampled label  */
    const float* teacher;          /* [n_tokens, k] Teacher log-probs         */
    const float* mask;             /* [n_tokens]                              */
    const float* rollout_lp;       /* [n_tokens], nullable                    */
    const int64_t* seg_offsets;    /* [n_docs + 2]                            */
    const int64_t* doc_ids;        /* [n_tokens], the ids seg_offsets is of   */
    int64_t n_tokens;
    int64_t n_docs;
    int64_t k;                     /* 1 <= k <= 256                           */
    int64_t n_docs_global;         /* MiniPlan.n_docs_global                  */
    int64_t n_tokens_global;       /* MiniPlan.n_tokens_global                */
    float lp_min_clamp;            /* log_prob_min_clamp (has_lp_clamp)       */
    float loss_max_clamp;          /* loss_max_clamp (has_loss_clamp)         */
    int32_t has_lp_clamp;
    int32_t has_loss_clamp;
    int32_t per_token_loss;        /* calculate_per_token_loss                */
    int32_t reserved;
    void* workspace;
    size_t workspace_bytes;
} meshy_distill_args;

size_t meshy_distill_workspace_size(int64_t n_tokens, int64_t n_docs);
/* out: [MESHY_DISTILL_NOUT] fp32 (device).  seg_cnt: [n_docs + 1] fp32
 * (device, nullable), the per-document mask counts the backward needs. */
int meshy_distill_loss_fwd(const meshy_distill_args* args, float* out, float* seg_cnt,
                           hipStream_t stream);
/* grad_student [n_tokens, k + 1]: d loss / d student * grad_loss[0] (device
 * scalar); column k (the sampled token, detached in the reference) is 0. */
int meshy_distill_loss_bwd(const meshy_distill_args* args, const float* seg_cnt,
                           const float* grad_loss, float* grad_student, hipStream_t stream);

/* forward_kl_topk alone (meshy/backend/titan/topk_loss.py:60-80), per
 * position i of n: kl[i] = sum_k exp(t) (t - s) over the k log-probs
 * student[i, :] and teacher[i, :] (contiguous [n, k]), both clamped from
 * below by lp_min_clamp when has_lp_clamp, the sum clamped to
 * [-loss_max_clamp, loss_max_clamp] when has_loss_clamp.  The backward
 * writes grad_student [n, k] = d kl / d student * grad_kl. */
int meshy_forward_kl_topk(const float* student, const float* teacher, int64_t n, int64_t k,
                          int32_t has_lp_clamp, float lp_min_clamp, int32_t has_loss_clamp,
                          float loss_max_clamp, float* kl, hipStream_t stream);
int meshy_forward_kl_topk_bwd(const float* student, const float* teacher, int64_t n, int64_t k,
                              int32_t has_lp_clamp, float lp_min_clamp, int32_t has_loss_clamp,
                              float loss_max_clamp, const float* grad_kl, float* grad_student,
                              hipStream_t stream);

/* ------------------------------------------------------------------------
 * Token-level clipped PPO loss with its diagnostics (device).
 * Replaces TitanTrainer._ppo_clip_loss (meshy/backend/titan/trainer.py:705-848)
 * and the per-mini sums _reduce_mini_metrics reads (trainer.py:1020-1047).
 *
 * Documents are contiguous token ranges: slot d covers tokens
 * [seg_offsets[d], seg_offsets[d+1]) of the flattened [rows, S] grid, for
 * d in [0, n_docs]; slot n_docs is the padding slot.  This is the segment
 * structure of doc_ids in both batch layouts (batch.py:123, 150-162).
 * ---------------------------------------------------------------------- */
enum meshy_ppo_out {
    MESHY_PPO_LOSS = 0,            /* pg loss (trainer.py:793-799)            */
    MESHY_PPO_TOTAL_LOSS,          /* loss + coef * positive_lm_loss          */
    MESHY_PPO_POSITIVE_LM_LOSS,
    MESHY_PPO_TIS_RATIO_SUM,
    MESHY_PPO_RATIO_SUM,
    MESHY_PPO_CLIP_SUM,
    MESHY_PPO_TIS_MASKED_SUM,
    MESHY_PPO_TOKEN_COUNT,
    MESHY_PPO_KL_SUM,
    MESHY_PPO_LOG_RATIO_ABS_SUM,
    MESHY_PPO_ESS_SUM,
    MESHY_PPO_DOC_COUNT,
    MESHY_PPO_TRAIN_ROLLOUT_KL_SUM,
    MESHY_PPO_TRAIN_ROLLOUT_LOGDIFF_ABS_SUM,
    MESHY_PPO_ENTROPY_SUM,
    MESHY_PPO_NOUT
};

typedef struct meshy_ppo_args {
    const float* new_lp;           /* [n_tokens]                              */
    const float* old_lp;           /* [n_tokens]                              */
    const float* mask;             /* [n_tokens]                              */
    const float* rollout_lp;       /* [n_tokens] nullable                     */
    const float* entropy;          /* [n_tokens] nullable                     */
    const float* adv;              /* [n_docs] or [n_tokens]                  */
    const float* positive_lm_weights; /* [n_docs], nullable                   */
    const int64_t* seg_offsets;    /* [n_docs + 2]                            */
    const int64_t* doc_ids;        /* [n_tokens], the ids seg_offsets is of   */
    float* grad_unit;              /* [n_tokens] nullable, see meshy_ppo_loss_fwd */
    int64_t n_tokens;
    int64_t n_docs;
    int64_t n_docs_global;         /* MiniPlan.n_docs_global                  */
    int64_t n_tokens_global;       /* MiniPlan.n_tokens_global                */
    float clip_low;                /* ppo_clip_eps_low                        */
    float clip_high;               /* ppo_clip_eps_high                       */
    float tis_min;
    float tis_max;
    float positive_lm_coef;
    int32_t adv_per_token;
    int32_t use_tis;
    int32_t use_icepop;
    int32_t per_token_loss;        /* calculate_per_token_loss                */
    int32_t train_lp_is_old;       /* old_logprobs_source == "train"          */
    int32_t cp_degree;
    int32_t reserved;
    void* workspace;
    size_t workspace_bytes;
} meshy_ppo_args;

/* Segment structure of a doc_ids tensor whose flattened values are
 * non-decreasing (both batch layouts, batch.py:123, 150-162):
 * seg_offsets[d] = number of tokens with id < d, for d in [0, n_slots].
 * unsorted (nullable, device int32) gets bit 1 when some doc_ids[i] >
 * doc_ids[i+1] and bit 2 when some id lies outside [0, n_slots - 1] (where
 * the reference's index_add_ raises); the caller clears it beforehand. */
int meshy_segment_offsets(const int64_t* doc_ids, int64_t n_tokens, int64_t n_slots,
                          int64_t* seg_offsets, int32_t* unsorted, hipStream_t stream);

size_t meshy_ppo_workspace_size(int64_t n_tokens, int64_t n_docs);
/* out: [MESHY_PPO_NOUT] fp32 (device).  seg_cnt: [n_docs + 1] fp32 (device,
 * nullable), the per-document masked token counts the sequence-mean backward
 * needs.  With the token-mean reduction (per_token_loss) and grad_unit set,
 * grad_unit[i] receives d(total loss)/d new_lp[i] at a unit loss gradient. */
int meshy_ppo_loss_fwd(const meshy_ppo_args* args, float* out, float* seg_cnt,
                       hipStream_t stream);
/* grad_new[i] = d(total loss)/d new_lp[i] * grad_loss[0]  (grad_loss is a
 * device scalar), matching torch autograd through trainer.py:751-809.  With
 * per_token_loss and grad_unit (as the forward filled it) this is
 * grad_loss[0] * grad_unit[i] and seg_cnt may be NULL; otherwise seg_cnt is
 * the forward's. */
int meshy_ppo_loss_bwd(const meshy_ppo_args* args, const float* seg_cnt,
                       const float* grad_loss, float* grad_new, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Segment-aware GAE and returns as a reverse affine scan (device).
 * Replaces compute_vapo_gae (meshy/backend/titan/critic/gae.py:208-293) and
 * compute_returns (gae.py:183-205), whose definition is the sequential loop
 * _reverse_scan_reference (gae.py:162-180) with the continuation rule of
 * _continuation_mask (gae.py:77-93) and the lambda rule of _lambda_per_doc
 * (gae.py:70-74).
 *
 * Inputs are [rows, S] row-major.  doc_ids in [0, n_docs] (n_docs = padding
 * slot).  values are fp32 (values_bf16 = 0) or bf16 (values_bf16 = 1).
 * lengths ([n_docs] fp32) may be NULL: each document's masked count is used.
 * seg_offsets ([n_docs + 2], nullable) are the segment offsets of doc_ids
 * (meshy_segment_offsets) when the flattened ids are non-decreasing, as in
 * both batch layouts: without lengths the masked counts are then fixed-order
 * sums (the same bits on every call, fractional masks included); without
 * offsets they are fp32 atomic sums, exact for 0/1 masks and order-dependent
 * in their last bits for fractional ones.
 * Outputs: adv [rows*S] (nullable), returns [rows*S] (nullable, decay gamma),
 * lam_doc [n_docs] (nullable).
 * ---------------------------------------------------------------------- */
typedef struct meshy_gae_args {
    const float* rewards;
    const void* values;            /* nullable when adv is NULL               */
    const float* mask;
    const int64_t* doc_ids;
    const float* lengths;
    int64_t rows;
    int64_t S;
    int64_t n_docs;
    float gamma;
    float alpha;
    float epsilon;
    int32_t values_bf16;
    float* adv;
    float* returns;
    float* lam_doc;
    void* workspace;
    size_t workspace_bytes;
    const int64_t* seg_offsets;    /* nullable, see above                     */
} meshy_gae_args;

size_t meshy_gae_workspace_size(int64_t rows, int64_t S, int64_t n_docs);
int meshy_gae(const meshy_gae_args* args, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Document order of unsorted doc_ids (device).
 * The reference sums per document with index_add_ over doc_ids in any order
 * (trainer.py:705-848 _ppo_clip_loss, opd.py:161-197 _distill_loss,
 * critic/gae.py:296-312 advantages_to_per_sequence); the kernels here take
 * each document as one run of tokens.  meshy_doc_order writes the stable sort
 * of the n token positions by document: perm[k] is the position of the k-th
 * token in document order (equal ids keep their order), sorted_ids[k] its id.
 * Every id must lie in [0, n_slots) (meshy_segment_offsets' range flag checks
 * it).  The workspace size comes from a query on the current device (0 when
 * it fails).
 * ---------------------------------------------------------------------- */
size_t meshy_doc_order_workspace_size(int64_t n, int64_t n_slots);
int meshy_doc_order(const int64_t* doc_ids, int64_t n, int64_t n_slots, int64_t* sorted_ids, int64_t* perm,
                    void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Test hook, no counterpart in the reference: the number of polls after which
 * meshy_gae's one-pass kernel stops waiting for a neighbouring chunk's map
 * and leaves the call to its exact fix-up pass (default 2000; a negative
 * limit restores it).  Returns the previous limit.  Process-wide; it applies
 * to calls launched after it (meshy_gae_attach included). */
int meshy_gae_set_poll_limit(int limit);

/* ------------------------------------------------------------------------
 * Per-token GAE advantages for a batch of samples (device).
 * Replaces TitanTrainer._attach_gae_advantages (meshy/backend/titan/trainer.py:603-699).
 * Samples are ragged: sample j covers [offsets[j], offsets[j+1]) of the flat
 * inputs, already cut to its width min(len, seq_len).  On the next-token grid
 * (trainer.py:656-667): mask[t] = mask_assistant[t+1] (0 at the sample's last
 * position), values as given, and the sample's reward at last - 1 where last
 * is its last position with mask_assistant > 0 (no reward when there is none
 * or last == 0).  lambda < 0 selects VAPO (lambda from each sample's masked
 * length with alpha); lambda in [0, 1] the constant-lambda rule with alpha = 1
 * and lengths 1 / max(1e-9, 1 - lambda) (trainer.py:669-683).
 * Outputs: adv [total] (zero outside the mask), grid_mask [total] (the
 * shifted mask, nullable), lam_doc [n] (nullable) and metrics [5] =
 * critic/value_mean, advantage_mean, advantage_abs_mean, advantage_seq_mean,
 * lambda_mean (trainer.py:688-699).
 * ---------------------------------------------------------------------- */
typedef struct meshy_gae_attach_args {
    const void* mask_assistant;    /* [total] fp32, or uint8 with mask_u8     */
    const void* values;            /* [total] fp32 or bf16                    */
    const float* reward;           /* [n]                                     */
    const int64_t* offsets;        /* [n + 1]                                 */
    int64_t n;
    int64_t total;
    float gamma;
    float alpha;
    float lambda;                  /* < 0: VAPO                               */
    float epsilon;
    int32_t values_bf16;
    int32_t mask_u8;               /* 1: mask_assistant holds bytes, each 0 or
                                      1 (meshy_host_gather_mask_u8)            */
    float* adv;                    /* [total]                                 */
    float* grid_mask;              /* [total], nullable                       */
    float* lam_doc;                /* [n], nullable                           */
    float* metrics;                /* [5], nullable                           */
    void* workspace;
    size_t workspace_bytes;
} meshy_gae_attach_args;

size_t meshy_gae_attach_workspace_size(int64_t n, int64_t total);
int meshy_gae_attach(const meshy_gae_attach_args* args, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Masked global whitening of per-token advantages (device).
 * Replaces the arithmetic of whiten_advantages (meshy/backend/titan/vapo.py:6-32):
 * fp64 sum / sum of squares / count over tokens with mask != 0, unbiased
 * variance (count >= 2), x <- (x - mean) * rsqrt(var + 1e-8) on the mask and
 * 0 elsewhere.  stats (device, [3] fp64) receives (sum, sumsq, count) before
 * the apply; `replication` divides them as the reference does before its
 * all-reduce.  Two phases so a caller can all-reduce `stats` in between:
 * meshy_whiten_stats then meshy_whiten_apply.
 * ---------------------------------------------------------------------- */
size_t meshy_whiten_workspace_size(int64_t n);
int meshy_whiten_stats(const float* adv, const float* mask, int64_t n, double replication,
                       double* stats, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);
int meshy_whiten_apply(float* adv, const float* mask, int64_t n, const double* stats,
                       hipStream_t stream);

/* ------------------------------------------------------------------------
 * Critic-side reductions (device).
 *
 * meshy_per_sequence_mean replaces advantages_to_per_sequence
 * (meshy/backend/titan/critic/gae.py:296-312): for each document d < n_docs,
 * out[d] = sum x[i] mask[i] / max(sum mask[i], 1) over its token range
 * [seg_offsets[d], seg_offsets[d+1]) (seg_offsets as for the PPO loss).
 *
 * meshy_critic_accumulate replaces Accumulator.update
 * (meshy/backend/titan/critic/metrics.py:238-275) on one [rows, S] row-major
 * micro-batch: with m = (mask > 0), v = values m (fp32 or bf16 values),
 * r = returns m, d = v - r, sums[0..4] (fp64, device) receive the sums of
 * m, r, r^2, d, d^2 and row_value[row] = sum_S v / max(sum_S m, 1).  The
 * workspace holds 5 doubles per row.
 *
 * meshy_clipped_value_error replaces clipped_value_error
 * (meshy/backend/titan/vapo.py:35-41): out = (v - t)^2, or with has_clip
 * max((v - t)^2, (o + clamp(v - o, -clip, clip) - t)^2); the backward gives
 * d out / d v * grad_out[i * grad_stride] (maximum splits ties, clamp passes
 * on its range); grad_stride 0 broadcasts one value, as the gradient of a sum
 * or a mean arrives, so it is never materialised.
 * ---------------------------------------------------------------------- */
int meshy_per_sequence_mean(const float* x, const float* mask, const int64_t* seg_offsets,
                            int64_t n_docs, float* out, hipStream_t stream);
size_t meshy_critic_accumulate_workspace_size(int64_t rows);
int meshy_critic_accumulate(const void* values, int32_t values_bf16, const float* returns,
                            const float* mask, int64_t rows, int64_t S, double* sums,
                            float* row_value, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);
int meshy_clipped_value_error(const float* values, const float* targets, const float* old_values,
                              int32_t has_clip, float clip, int64_t n, float* out,
                              hipStream_t stream);

/* ------------------------------------------------------------------------
 * Critic gauges of one window (device).
 *
 * meshy_critic_window_sums: the token-level part of critic_diagnostics
 * (meshy/backend/titan/critic/metrics.py:189-217) over a [rows, S] row-major
 * window, with the mask m as given (fractional values included).  With
 * e = v - r (fp32), sel = (m > 0):
 *   sums[MESHY_CW_SEL]    #sel                sums[MESHY_CW_M]    sum m
 *   sums[MESHY_CW_R]      sum_sel r           sums[MESHY_CW_E2M]  sum e^2 m
 *   sums[MESHY_CW_R2]     sum_sel r^2         sums[MESHY_CW_EM]   sum e m
 *   sums[MESHY_CW_D]      sum_sel e           sums[MESHY_CW_RMIN] min_sel r
 *   sums[MESHY_CW_D2]     sum_sel e^2         sums[MESHY_CW_RMAX] max_sel r
 * (fp64, device; the sel sums select, as variance_reduction does, metrics.py:
 * 120-138; the m sums multiply, as the loss and calibration_gap do), and
 * row_value[row] = sum_S v m / max(sum_S m, 1) (_response_mean, 58-62).
 * Workspace: MESHY_CW_VALS doubles per row.  Rows are reduced in a fixed
 * order: the same bits on every call.
 *
 * meshy_group_gauges: within_prompt_auc (metrics.py:94-118) and prompt_pearson
 * (64-91) over n rows in any order, grouped by group_ids.  A row is correct
 * when row_reward >= correct_threshold.  out[0] = wins (pairs of a correct and
 * an incorrect row of one group where the correct one's value is greater, ties
 * counting 1/2), out[1] = such pairs, out[2] = groups, out[3] = Pearson r of
 * the groups' mean value against their mean reward (NaN for fewer than two
 * groups or a constant side).  The AUC is out[0] / out[1] (NaN without
 * pairs).  O(n^2) pair checks (n is a window's row count); workspace 5
 * doubles per row; fixed-order reductions.
 * ---------------------------------------------------------------------- */
enum {
    MESHY_CW_SEL = 0, MESHY_CW_R, MESHY_CW_R2, MESHY_CW_D, MESHY_CW_D2,
    MESHY_CW_M, MESHY_CW_E2M, MESHY_CW_EM, MESHY_CW_RMIN, MESHY_CW_RMAX,
    MESHY_CW_VALS
};
size_t meshy_critic_window_workspace_size(int64_t rows);
int meshy_critic_window_sums(const void* values, int32_t values_bf16, const float* returns,
                             const float* mask, int64_t rows, int64_t S, double* sums,
                             float* row_value, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);
size_t meshy_group_gauges_workspace_size(int64_t n);
int meshy_group_gauges(const float* row_value, const float* row_reward, const int64_t* group_ids,
                       int64_t n, float correct_threshold, double* out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);
int meshy_clipped_value_error_bwd(const float* values, const float* targets,
                                  const float* old_values, int32_t has_clip, float clip, int64_t n,
                                  const float* grad_out, int64_t grad_stride, float* grad_values,
                                  hipStream_t stream);

/* ------------------------------------------------------------------------
 * Token-level rollout statistics over jagged sample columns (device).
 * Replaces the per-token loops of TitanTrainer._rollout_metrics
 * (meshy/backend/titan/metrics.py:197-212).  Sample s covers
 * mask[offsets[s] .. offsets[s+1]) and logprobs[lp_offsets[s] ..
 * lp_offsets[s+1]) (the values() / offsets() of jagged nested columns).
 *   resp_len[s]  #(mask > 0)
 *   lp_sum[s]    sum of the kept log-probs (fp64): those with mask > 0 when
 *                the sample's log-prob column is as long as its mask, else all
 *   out_off      [n + 1] exclusive scan of the kept counts (required)
 *   kept_lp      the kept log-probs in sample order (nullable; room for every
 *                log-prob is enough)
 * logprobs may be NULL (no log-prob column).  Workspace: one int64 per sample.
 * ---------------------------------------------------------------------- */
size_t meshy_ragged_token_stats_workspace_size(int64_t n);
int meshy_ragged_token_stats(const float* mask, const float* logprobs, const int64_t* offsets,
                             const int64_t* lp_offsets, int64_t n, int64_t* resp_len,
                             double* lp_sum, int64_t* out_off, float* kept_lp, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Measurement helper; no counterpart in the reference.  Streams rows x
 * row_bytes bytes from src (one workgroup per row, 16-byte nontemporal loads,
 * 8 in flight per thread, the access pattern of meshy_logprob_entropy_fwd)
 * and folds them into out[0], so a benchmark can report the read bandwidth
 * this device reaches on that pattern next to the kernels' figures.
 * row_bytes must be a multiple of 16 and src 16-byte aligned.
 * ---------------------------------------------------------------------- */
int meshy_stream_read(const void* src, int64_t rows, int64_t row_bytes, uint32_t* out,
                      hipStream_t stream);

/* ------------------------------------------------------------------------
 * Counter-based synthetic bf16 logits drawn from N(0, scale^2) (device and
 * host, the same bits).  No reference counterpart: the synthetic inputs of
 * the measured workloads, regenerated on the host for the rows a parity
 * check reads, instead of copying a tensor of up to 34 GB.  Elements 2p and
 * 2p + 1 (element k = row * cols + col) are the Box-Muller pair of
 *   h = mix(mix(seed) ^ p), mix = splitmix64's finaliser:
 *   u1 = (lo32(h) + 1) / 2^32, theta = 2 pi hi32(h) / 2^32,
 *   scale * sqrt(-2 ln u1) * (cos theta, sin theta),
 * each rounded to bf16 (nearest even).  The fp32 log, square root, sine and
 * cosine are the library's own, built from correctly rounded adds,
 * multiplies and fused multiply-adds only, so both sides give the same bits;
 * |value| <= 6.66 scale.
 * meshy_synth_bf16 fills out[row * row_stride + col] for a [rows, cols]
 * block on the stream; meshy_synth_bf16_rows_host writes rows row_ids[i] of
 * the same block to out[i * cols ...] on host threads.
 * ---------------------------------------------------------------------- */
int meshy_synth_bf16(uint16_t* out, int64_t rows, int64_t cols, int64_t row_stride, uint64_t seed, float scale,
                     hipStream_t stream);
int meshy_synth_bf16_rows_host(uint16_t* out, const int64_t* row_ids, int64_t n_rows, int64_t cols,
                               uint64_t seed, float scale);

#ifdef __cplusplus
}
#endif

#endif /* MESHY_AMD_H */
