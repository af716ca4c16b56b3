// Token-budget planner, host side.
//
// Produces the same assignment as build_plan (meshy/backend/titan/plan.py:211-288):
//   1. truncate lengths to seq_len (plan.py:237);
//   2. order samples by (-length, index) and deal them boustrophedon over the
//      DP ranks (plan.py:240-241, _snake plan.py:145-155);
//   3. per rank, deal the rank's samples boustrophedon over the mini-batches
//      (plan.py:249-257), then first-fit-decreasing into micro-batches
//      (_pack_micros plan.py:158-203);
//   4. pad every mini-batch index to the same micro count with fillers and
//      attach the global loss denominators (plan.py:259-283).
// The output is a set of flat CSR tables (see meshy_plan_out in meshy_amd.h).
// The sort of step 2 is a stable radix sort by length (its input is in index
// order, so ties stay in index order), and the first fit of step 3 a descent
// of a max-tree over the open micros' free capacities: O(n log m) where the
// reference's scan of every open micro is O(n m).
#include <algorithm>
#include <climits>
#include <cmath>
#include <new>
#include <vector>

#include "host_common.h"

namespace {

using meshy::set_error;

inline int64_t round_up(int64_t x, int64_t align) { return ((x + align - 1) / align) * align; }

// Boustrophedon deal of `order` into n_bins bins (plan.py:145-155).
std::vector<std::vector<int64_t>> snake(const std::vector<int64_t>& order, int64_t n_bins) {
    std::vector<std::vector<int64_t>> bins(static_cast<size_t>(n_bins));
    for (size_t k = 0; k < order.size(); ++k) {
        const int64_t rnd = static_cast<int64_t>(k) / n_bins;
        const int64_t pos = static_cast<int64_t>(k) % n_bins;
        const int64_t bin = (rnd % 2 == 0) ? pos : n_bins - 1 - pos;
        bins[static_cast<size_t>(bin)].push_back(order[k]);
    }
    return bins;
}

// Positions ordered by (-len[p], p), the reference's sort key (plan.py:164, 240).
bool in_length_order(const std::vector<int64_t>& order, const std::vector<int64_t>& len) {
    for (size_t k = 1; k < order.size(); ++k) {
        const int64_t a = order[k - 1], b = order[k];
        if (len[a] < len[b] || (len[a] == len[b] && a > b)) return false;
    }
    return true;
}

// Stable LSD radix sort of `order` by decreasing length, 11 bits of the
// length's distance below the maximum per pass: ties keep their input order.
void radix_by_length_desc(std::vector<int64_t>& order, const std::vector<int64_t>& len, int64_t hi,
                          uint64_t range) {
    constexpr int kBits = 11;
    constexpr uint64_t kMask = (uint64_t{1} << kBits) - 1;
    std::vector<int64_t> tmp(order.size());
    std::vector<uint32_t> cnt(size_t{1} << kBits);
    for (int shift = 0; shift == 0 || (shift < 64 && (range >> shift) != 0); shift += kBits) {
        std::fill(cnt.begin(), cnt.end(), 0u);
        for (int64_t p : order) ++cnt[(static_cast<uint64_t>(hi - len[p]) >> shift) & kMask];
        uint32_t run = 0;
        for (uint32_t& c : cnt) {
            const uint32_t v = c;
            c = run;
            run += v;
        }
        for (int64_t p : order) tmp[cnt[(static_cast<uint64_t>(hi - len[p]) >> shift) & kMask]++] = p;
        order.swap(tmp);
    }
}

std::vector<int64_t> by_length_desc(const std::vector<int64_t>& idx, const std::vector<int64_t>& len,
                                    bool ascending_input) {
    std::vector<int64_t> order(idx);
    if (order.size() < 2 || in_length_order(order, len)) return order;
    int64_t lo = len[order[0]], hi = lo;
    for (int64_t p : order) {
        lo = std::min(lo, len[p]);
        hi = std::max(hi, len[p]);
    }
    // hi - lo overflows only for lengths of opposite signs beyond 2^62.
    const bool small_range = lo >= -(int64_t{1} << 62) && hi <= (int64_t{1} << 62);
    if (ascending_input && small_range && order.size() >= 256 && order.size() < UINT32_MAX) {
        radix_by_length_desc(order, len, hi, static_cast<uint64_t>(hi - lo));
        return order;
    }
    std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        if (len[a] != len[b]) return len[a] > len[b];
        return a < b;
    });
    return order;
}

// Indices 0..n-1 ordered by (-len[i], i).
std::vector<int64_t> by_length_desc(const std::vector<int64_t>& len) {
    std::vector<int64_t> idx(len.size());
    for (size_t i = 0; i < idx.size(); ++i) idx[i] = static_cast<int64_t>(i);
    return by_length_desc(idx, len, true);
}

// The micros of one mini-batch as flat tables: micro j holds the samples
// pos[start[j] .. start[j + 1]) (rank-local positions, truncated lengths in
// lens) and pads to seq_len[j].
struct Micros {
    std::vector<int64_t> seq_len;
    std::vector<int64_t> start;
    std::vector<int64_t> pos;
    std::vector<int64_t> lens;
    size_t size() const { return seq_len.size(); }
};

// The leftmost of the open micros (creation order) whose free capacity is at
// least `need`, through a max-tree over the capacities: first-fit in O(log m)
// per sample instead of a scan of every open micro.
class FirstFit {
   public:
    int64_t find(int64_t need) const {
        if (count_ == 0 || tree_[1] < need) return -1;
        size_t node = 1;
        // Branch-free descent: left child when it holds a fit, else right.
        while (node < leaves_) node = 2 * node + static_cast<size_t>(tree_[2 * node] < need);
        return static_cast<int64_t>(node - leaves_);
    }
    // Stops climbing where a node's maximum is unchanged.
    void set(int64_t i, int64_t cap) {
        size_t node = leaves_ + static_cast<size_t>(i);
        tree_[node] = cap;
        for (node >>= 1; node > 0; node >>= 1) {
            const int64_t m = std::max(tree_[2 * node], tree_[2 * node + 1]);
            if (tree_[node] == m) break;
            tree_[node] = m;
        }
    }
    int64_t push(int64_t cap) {
        if (count_ == leaves_) grow();
        set(static_cast<int64_t>(count_), cap);
        return static_cast<int64_t>(count_++);
    }

   private:
    static constexpr int64_t kNone = INT64_MIN;  // an unused leaf: never fits
    void grow() {
        const size_t nl = leaves_ ? 2 * leaves_ : 16;
        std::vector<int64_t> t(2 * nl, kNone);
        for (size_t i = 0; i < count_; ++i) t[nl + i] = tree_[leaves_ + i];
        for (size_t node = nl - 1; node > 0; --node) t[node] = std::max(t[2 * node], t[2 * node + 1]);
        tree_.swap(t);
        leaves_ = nl;
    }
    std::vector<int64_t> tree_;
    size_t leaves_ = 0;
    size_t count_ = 0;
};

// First-fit-decreasing of `members` (rank-local positions) into micros
// (plan.py:158-203).  A micro's admission test is a capacity against a need:
//   packed:  round_up(total + L, align) <= budget  <=>  total + L <= floor(budget / align) * align,
//            capacity floor(budget / align) * align - total, need L;
//   padded:  (rows + 1) * row_len <= budget  <=>  rows + 1 <= floor(budget / row_len),
//            or rows < micro_batch_size without a budget: capacity in rows, need 1.
// Both forms keep the reference's choice, the first open micro that passes.
Micros pack_micros(const std::vector<int64_t>& members,
                               const std::vector<int64_t>& local_len,
                               const meshy_planner_cfg& cfg) {
    // The members arrive in this order from the deal; the check keeps the
    // sort for any other caller.
    const std::vector<int64_t> order = by_length_desc(members, local_len, false);
    const bool padded = cfg.layout == MESHY_LAYOUT_PADDED;
    const bool has_budget = cfg.max_tokens_per_micro > 0;
    const int64_t budget = cfg.max_tokens_per_micro;
    // The row cap applies only without a token budget (plan.py:166-168).
    const int64_t max_rows = cfg.micro_batch_size;
    const int64_t packed_cap = has_budget ? budget / cfg.align * cfg.align : 0;

    std::vector<int64_t> acc;   // padded: row length fixed by the first sample; packed: token total
    std::vector<int64_t> rows;  // samples in the micro
    std::vector<int64_t> max_rows_of;  // padded: rows the micro admits
    std::vector<int64_t> micro_of(order.size());
    FirstFit fit;
    for (size_t k = 0; k < order.size(); ++k) {
        const int64_t L = local_len[order[k]];
        const int64_t j = fit.find(padded ? 1 : L);
        if (j >= 0) {
            micro_of[k] = j;
            ++rows[j];
            if (padded) {
                fit.set(j, max_rows_of[j] - rows[j]);
            } else {
                acc[j] += L;
                fit.set(j, packed_cap - acc[j]);
            }
        } else {
            const int64_t a = padded ? round_up(L, cfg.align) : L;
            int64_t cap;
            if (padded) {
                const int64_t mr = has_budget ? (a > 0 ? budget / a : INT64_MAX) : max_rows;
                max_rows_of.push_back(mr);
                cap = mr - 1;
            } else {
                max_rows_of.push_back(0);
                cap = packed_cap - a;
            }
            micro_of[k] = fit.push(cap);
            acc.push_back(a);
            rows.push_back(1);
        }
    }
    // Bucket the samples by micro, in placement order within each.
    const size_t m = acc.size();
    Micros out;
    out.seq_len.resize(m);
    out.start.assign(m + 1, 0);
    for (size_t j = 0; j < m; ++j) {
        out.seq_len[j] = padded ? acc[j] : round_up(acc[j], cfg.align);
        out.start[j + 1] = out.start[j] + rows[j];
    }
    out.pos.resize(order.size());
    out.lens.resize(order.size());
    std::vector<int64_t> fill(out.start.begin(), out.start.end() - 1);
    for (size_t k = 0; k < order.size(); ++k) {
        const int64_t at = fill[static_cast<size_t>(micro_of[k])]++;
        out.pos[at] = order[k];
        out.lens[at] = local_len[order[k]];
    }
    return out;
}

int plan_impl(const int64_t* lengths, const int64_t* loss_tokens, int64_t n, int64_t dp,
              const meshy_planner_cfg& cfg, meshy_plan_out* out) {
    if (n == 0) return set_error(MESHY_EEMPTY, "cannot plan an empty batch");
    if (dp <= 0 || n % dp != 0) {
        return set_error(MESHY_ENOTDIV,
                         "batch size %lld is not divisible by DP size %lld; adjust "
                         "rollout.batch_size * group_size to a multiple of dp_replicate * dp_shard",
                         static_cast<long long>(n), static_cast<long long>(dp));
    }
    if (cfg.layout != MESHY_LAYOUT_PADDED && cfg.layout != MESHY_LAYOUT_PACKED)
        return set_error(MESHY_EINVAL, "unknown layout %d", cfg.layout);
    if (cfg.mini_batch_size <= 0) return set_error(MESHY_EINVAL, "mini_batch_size must be positive");
    if (cfg.align <= 0 || cfg.seq_len <= 0)
        return set_error(MESHY_EINVAL, "align and seq_len must be positive");
    if (cfg.max_tokens_per_micro <= 0 && cfg.micro_batch_size <= 0)
        return set_error(MESHY_EINVAL, "either max_tokens_per_micro or micro_batch_size must be set");
    if (cfg.layout == MESHY_LAYOUT_PACKED && cfg.max_tokens_per_micro <= 0)
        return set_error(MESHY_EINVAL, "packed layout requires max_tokens_per_micro");

    std::vector<int64_t> trunc(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) trunc[i] = std::min(lengths[i], cfg.seq_len);

    // 1. DP partition (plan.py:239-243).
    const std::vector<int64_t> order = by_length_desc(trunc);
    const std::vector<std::vector<int64_t>> rank_samples = snake(order, dp);
    const int64_t n_local = n / dp;
    const int64_t n_mini = (n_local + cfg.mini_batch_size - 1) / cfg.mini_batch_size;

    // 2. Per rank: minis by snake, micros by first-fit-decreasing (plan.py:247-257).
    std::vector<std::vector<std::vector<int64_t>>> members(static_cast<size_t>(dp));
    std::vector<std::vector<Micros>> minis(static_cast<size_t>(dp));
    for (int64_t r = 0; r < dp; ++r) {
        const std::vector<int64_t>& local = rank_samples[r];
        std::vector<int64_t> local_len(local.size());
        for (size_t p = 0; p < local.size(); ++p) local_len[p] = trunc[local[p]];
        members[r] = snake(by_length_desc(local_len), n_mini);
        minis[r].reserve(static_cast<size_t>(n_mini));
        for (int64_t i = 0; i < n_mini; ++i) minis[r].push_back(pack_micros(members[r][i], local_len, cfg));
    }

    // 3. Equalise micro counts and attach global denominators (plan.py:259-283).
    int64_t n_micro_total = 0;
    for (int64_t i = 0; i < n_mini; ++i) {
        size_t n_micro = 0;
        int64_t n_docs_global = 0;
        int64_t n_tokens_global = 0;
        for (int64_t q = 0; q < dp; ++q) {
            n_micro = std::max(n_micro, minis[q][i].size());
            n_docs_global += static_cast<int64_t>(members[q][i].size());
            int64_t tokens_q = 0;
            for (int64_t p : members[q][i]) {
                const int64_t g = rank_samples[q][p];
                n_tokens_global += loss_tokens[g];
                tokens_q += trunc[g];
            }
            out->mini_tokens_per_rank[i * dp + q] = tokens_q;
        }
        out->mini_n_micro[i] = static_cast<int32_t>(n_micro);
        out->mini_n_docs_global[i] = n_docs_global;
        out->mini_n_tokens_global[i] = n_tokens_global;
        n_micro_total += static_cast<int64_t>(n_micro);
    }

    for (int64_t r = 0; r < dp; ++r) {
        for (int64_t p = 0; p < n_local; ++p) out->local_indices[r * n_local + p] = static_cast<int32_t>(rank_samples[r][p]);
        int64_t k = 0;
        int32_t cursor = 0;
        int64_t* seq = out->micro_seq_len + r * n_local;
        int32_t* start = out->micro_doc_start + r * (n_local + 1);
        int32_t* dsample = out->doc_sample + r * n_local;
        int64_t* dlen = out->doc_len + r * n_local;
        for (int64_t i = 0; i < n_mini; ++i) {
            const Micros& ms = minis[r][i];
            const int64_t n_micro = out->mini_n_micro[i];
            for (int64_t j = 0; j < n_micro; ++j, ++k) {
                start[k] = cursor;
                if (j < static_cast<int64_t>(ms.size())) {
                    seq[k] = ms.seq_len[j];
                    for (int64_t d = ms.start[j]; d < ms.start[j + 1]; ++d, ++cursor) {
                        dsample[cursor] = static_cast<int32_t>(ms.pos[d]);
                        dlen[cursor] = ms.lens[d];
                    }
                } else {
                    seq[k] = cfg.align;  // filler micro (plan.py:206-208)
                }
            }
        }
        start[k] = cursor;
    }
    out->n_micro_total = static_cast<int32_t>(n_micro_total);
    return MESHY_OK;
}

}  // namespace

namespace {

// #(m[t] > 0) over n floats; branch-free so it vectorises, with an AVX2 form
// picked at load time where the CPU has it.
__attribute__((target_clones("avx2", "default"))) int64_t count_positive(const float* m, int64_t n) {
    int32_t c = 0;
    for (int64_t t = 0; t < n; ++t) c += static_cast<int32_t>(m[t] > 0.f);
    return c;
}

// The same over a mask of bytes (each 0 or 1, or any byte: nonzero counts).
__attribute__((target_clones("avx2", "default"))) int64_t count_positive(const uint8_t* m, int64_t n) {
    int32_t c = 0;
    for (int64_t t = 0; t < n; ++t) c += static_cast<int32_t>(m[t] != 0);
    return c;
}

template <typename M>
int sample_loss_tokens(const char* who, const M* mask, const int64_t* offsets, int64_t n, int64_t seq_len,
                       int64_t* lengths, int64_t* loss_tokens) {
    if (n < 0 || seq_len <= 0) return set_error(MESHY_EINVAL, "%s: bad sizes", who);
    if (n > 0 && (!offsets || !lengths || !loss_tokens || (!mask && offsets[n] > offsets[0])))
        return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    for (int64_t i = 0; i < n; ++i) {
        const int64_t a = offsets[i];
        const int64_t len = offsets[i + 1] - a;
        if (len < 0) return set_error(MESHY_EINVAL, "%s: offsets decrease at %lld", who, static_cast<long long>(i));
        lengths[i] = len;
        const int64_t L = std::min(len, seq_len);
        loss_tokens[i] = L > 1 ? count_positive(mask + a + 1, L - 1) : 0;
    }
    return MESHY_OK;
}

}  // namespace

extern "C" int meshy_sample_loss_tokens(const float* mask, const int64_t* offsets, int64_t n,
                                        int64_t seq_len, int64_t* lengths, int64_t* loss_tokens) {
    meshy::clear_error();
    return sample_loss_tokens("meshy_sample_loss_tokens", mask, offsets, n, seq_len, lengths, loss_tokens);
}

extern "C" int meshy_sample_loss_tokens_u8(const uint8_t* mask, const int64_t* offsets, int64_t n,
                                           int64_t seq_len, int64_t* lengths, int64_t* loss_tokens) {
    meshy::clear_error();
    return sample_loss_tokens("meshy_sample_loss_tokens_u8", mask, offsets, n, seq_len, lengths, loss_tokens);
}

// GRPO advantages of host rewards: per group (offsets clamped to the rewards
// as the device kernel clamps them) a size-1 group keeps its reward, any other
// gets (r - mean) / max(unbiased std, 1e-8), in fp32 like the reference's
// torch arithmetic, with the two sums taken in fp64.
extern "C" int meshy_grpo_advantage_host(const float* rewards, int64_t n_rewards, const int64_t* group_offsets,
                                         int64_t n_groups, float* advantages) {
    meshy::clear_error();
    if (n_groups < 0 || n_rewards < 0) return set_error(MESHY_EINVAL, "meshy_grpo_advantage_host: negative count");
    if (n_groups == 0) return MESHY_OK;
    if ((!rewards && n_rewards > 0) || !group_offsets || (!advantages && n_rewards > 0))
        return set_error(MESHY_ENULL, "meshy_grpo_advantage_host: NULL pointer");
    for (int64_t g = 0; g < n_groups; ++g) {
        const int64_t b = std::min(std::max(group_offsets[g], static_cast<int64_t>(0)), n_rewards);
        const int64_t e = std::min(std::max(group_offsets[g + 1], b), n_rewards);
        const int64_t n = e - b;
        if (n <= 0) continue;
        if (n == 1) {
            advantages[b] = rewards[b];
            continue;
        }
        double sum = 0.0;
        for (int64_t i = b; i < e; ++i) sum += rewards[i];
        const float mean = static_cast<float>(sum / static_cast<double>(n));
        double sq = 0.0;
        for (int64_t i = b; i < e; ++i) {
            const double d = static_cast<double>(rewards[i] - mean);
            sq += d * d;
        }
        const float sd = static_cast<float>(std::sqrt(sq / static_cast<double>(n - 1)));
        const float den = std::max(sd, 1e-8f);
        for (int64_t i = b; i < e; ++i) advantages[i] = (rewards[i] - mean) / den;
    }
    return MESHY_OK;
}

// Python's max()/min() over the group (a NaN first element stays, later NaNs
// lose every comparison), then the spread against the tolerance; offsets are
// clamped to the rewards as the device filter clamps them.
extern "C" int meshy_zero_variance_groups_host(const double* raw_rewards, int64_t n_rewards,
                                               const int64_t* group_offsets, int64_t n_groups, double tolerance,
                                               uint8_t* flags) {
    meshy::clear_error();
    if (n_groups < 0 || n_rewards < 0)
        return set_error(MESHY_EINVAL, "meshy_zero_variance_groups_host: negative count");
    if (n_groups == 0) return MESHY_OK;
    if ((!raw_rewards && n_rewards > 0) || !group_offsets || !flags)
        return set_error(MESHY_ENULL, "meshy_zero_variance_groups_host: NULL pointer");
    for (int64_t g = 0; g < n_groups; ++g) {
        const int64_t b = std::min(std::max(group_offsets[g], static_cast<int64_t>(0)), n_rewards);
        const int64_t e = std::min(std::max(group_offsets[g + 1], b), n_rewards);
        if (e <= b) {
            flags[g] = 1;
            continue;
        }
        double hi = raw_rewards[b], lo = raw_rewards[b];
        for (int64_t i = b + 1; i < e; ++i) {
            const double r = raw_rewards[i];
            if (r > hi) hi = r;
            if (r < lo) lo = r;
        }
        flags[g] = static_cast<uint8_t>(hi - lo <= tolerance);
    }
    return MESHY_OK;
}

extern "C" int meshy_plan_build(const int64_t* lengths, const int64_t* loss_tokens, int64_t n,
                                int64_t dp_size, const meshy_planner_cfg* cfg, meshy_plan_out* out) {
    meshy::clear_error();
    if (!cfg || !out) return set_error(MESHY_ENULL, "meshy_plan_build: cfg and out are required");
    if (n < 0) return set_error(MESHY_EINVAL, "meshy_plan_build: negative sample count");
    if (n > 0 && (!lengths || !loss_tokens))
        return set_error(MESHY_ENULL, "meshy_plan_build: lengths and loss_tokens are required");
    if (n > 0 && dp_size > 0 && n % dp_size == 0 && cfg->mini_batch_size > 0 &&
        (!out->local_indices || !out->mini_n_micro || !out->mini_n_docs_global ||
         !out->mini_n_tokens_global || !out->mini_tokens_per_rank || !out->micro_seq_len ||
         !out->micro_doc_start || !out->doc_sample || !out->doc_len))
        return set_error(MESHY_ENULL, "meshy_plan_build: every output table is required");
    if (n > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_plan_build: too many samples");
    try {
        return plan_impl(lengths, loss_tokens, n, dp_size, *cfg, out);
    } catch (const std::bad_alloc&) {
        return set_error(MESHY_EINVAL, "meshy_plan_build: out of host memory");
    }
}

extern "C" int meshy_step_plan(meshy_step_plan_args* args) {
    meshy::clear_error();
    if (!args) return set_error(MESHY_ENULL, "meshy_step_plan: args is NULL");
    meshy_step_plan_args& a = *args;
    if (a.n <= 0) return set_error(MESHY_EEMPTY, "cannot plan an empty batch");
    if (a.dp_size <= 0 || a.rank < 0 || a.rank >= a.dp_size)
        return set_error(MESHY_EINVAL, "meshy_step_plan: rank %lld outside %lld ranks",
                         static_cast<long long>(a.rank), static_cast<long long>(a.dp_size));
    if (!a.micro_seq_len || !a.micro_out_off || !a.micro_doc_start || !a.doc_sample || !a.doc_len)
        return set_error(MESHY_ENULL, "meshy_step_plan: every pack table is required");
    int rc = a.mask_u8 ? sample_loss_tokens("meshy_step_plan", static_cast<const uint8_t*>(a.mask), a.offsets, a.n,
                                            a.cfg.seq_len, a.lengths, a.loss_tokens)
                       : sample_loss_tokens("meshy_step_plan", static_cast<const float*>(a.mask), a.offsets, a.n,
                                            a.cfg.seq_len, a.lengths, a.loss_tokens);
    if (rc) return rc;
    rc = meshy_plan_build(a.lengths, a.loss_tokens, a.n, a.dp_size, &a.cfg, &a.plan);
    if (rc) return rc;
    // The rank's slice of the planner's tables, as the pack reads them.
    const int64_t n_local = a.n / a.dp_size;
    const int64_t nm = a.plan.n_micro_total;
    const int64_t* seq = a.plan.micro_seq_len + a.rank * n_local;
    const int32_t* start = a.plan.micro_doc_start + a.rank * (n_local + 1);
    const int32_t* local = a.plan.local_indices + a.rank * n_local;
    const int32_t* dsample = a.plan.doc_sample + a.rank * n_local;
    const int64_t* dlen = a.plan.doc_len + a.rank * n_local;
    const bool packed = a.cfg.layout == MESHY_LAYOUT_PACKED;
    int64_t off = 0, max_elems = 0, max_docs = 0;
    a.micro_out_off[0] = 0;
    for (int64_t k = 0; k < nm; ++k) {
        const int64_t docs = static_cast<int64_t>(start[k + 1]) - start[k];
        const int64_t elems = seq[k] * (packed ? 1 : std::max<int64_t>(docs, 1));
        a.micro_seq_len[k] = seq[k];
        a.micro_doc_start[k] = start[k];
        off += elems;
        a.micro_out_off[k + 1] = off;
        max_elems = std::max(max_elems, elems);
        max_docs = std::max(max_docs, docs);
    }
    a.micro_doc_start[nm] = start[nm];
    const int64_t nd = start[nm];
    for (int64_t j = 0; j < nd; ++j) {
        a.doc_sample[j] = local[dsample[j]];
        a.doc_len[j] = dlen[j];
    }
    a.n_micro = nm;
    a.n_docs = nd;
    a.max_micro_elems = max_elems;
    a.max_docs_per_micro = max_docs;
    return MESHY_OK;
}
