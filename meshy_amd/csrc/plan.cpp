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
#include <algorithm>
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

// Indices 0..n-1 ordered by (-len[i], i).
std::vector<int64_t> by_length_desc(const std::vector<int64_t>& len) {
    std::vector<int64_t> order(len.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<int64_t>(i);
    std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        if (len[a] != len[b]) return len[a] > len[b];
        return a < b;
    });
    return order;
}

struct Micro {
    std::vector<int64_t> pos;   // rank-local sample positions
    std::vector<int64_t> lens;  // truncated lengths
    int64_t seq_len;
};

// First-fit-decreasing of `members` (rank-local positions) into micros
// (plan.py:158-203).
std::vector<Micro> pack_micros(const std::vector<int64_t>& members,
                               const std::vector<int64_t>& local_len,
                               const meshy_planner_cfg& cfg) {
    std::vector<int64_t> order(members);
    std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        if (local_len[a] != local_len[b]) return local_len[a] > local_len[b];
        return a < b;
    });
    const bool padded = cfg.layout == MESHY_LAYOUT_PADDED;
    const bool has_budget = cfg.max_tokens_per_micro > 0;
    const int64_t budget = cfg.max_tokens_per_micro;
    // The row cap applies only without a token budget (plan.py:166-168).
    const bool has_row_cap = !has_budget && cfg.micro_batch_size > 0;
    const int64_t max_rows = cfg.micro_batch_size;

    struct Open {
        std::vector<int64_t> pos;
        std::vector<int64_t> lens;
        int64_t acc;  // padded: row length fixed by the first sample; packed: token total
    };
    std::vector<Open> open;
    for (int64_t p : order) {
        const int64_t L = local_len[p];
        bool placed = false;
        for (Open& m : open) {
            const int64_t rows = static_cast<int64_t>(m.pos.size());
            if (has_row_cap && rows >= max_rows) continue;
            if (has_budget) {
                const int64_t cost = padded ? (rows + 1) * m.acc : round_up(m.acc + L, cfg.align);
                if (cost > budget) continue;
            }
            m.pos.push_back(p);
            m.lens.push_back(L);
            if (!padded) m.acc += L;
            placed = true;
            break;
        }
        if (!placed) {
            Open m;
            m.pos.push_back(p);
            m.lens.push_back(L);
            m.acc = padded ? round_up(L, cfg.align) : L;
            open.push_back(std::move(m));
        }
    }
    std::vector<Micro> out;
    out.reserve(open.size());
    for (Open& m : open) {
        Micro mp;
        mp.seq_len = padded ? m.acc : round_up(m.acc, cfg.align);
        mp.pos = std::move(m.pos);
        mp.lens = std::move(m.lens);
        out.push_back(std::move(mp));
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
    std::vector<std::vector<std::vector<Micro>>> minis(static_cast<size_t>(dp));
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
            const std::vector<Micro>& ms = minis[r][i];
            const int64_t n_micro = out->mini_n_micro[i];
            for (int64_t j = 0; j < n_micro; ++j, ++k) {
                start[k] = cursor;
                if (j < static_cast<int64_t>(ms.size())) {
                    seq[k] = ms[j].seq_len;
                    for (size_t d = 0; d < ms[j].pos.size(); ++d, ++cursor) {
                        dsample[cursor] = static_cast<int32_t>(ms[j].pos[d]);
                        dlen[cursor] = ms[j].lens[d];
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

extern "C" int meshy_sample_loss_tokens(const float* mask, const int64_t* offsets, int64_t n,
                                        int64_t seq_len, int64_t* lengths, int64_t* loss_tokens) {
    meshy::clear_error();
    if (n < 0 || seq_len <= 0) return set_error(MESHY_EINVAL, "meshy_sample_loss_tokens: bad sizes");
    if (n > 0 && (!offsets || !lengths || !loss_tokens || (!mask && offsets[n] > offsets[0])))
        return set_error(MESHY_ENULL, "meshy_sample_loss_tokens: NULL pointer");
    for (int64_t i = 0; i < n; ++i) {
        const int64_t a = offsets[i];
        const int64_t len = offsets[i + 1] - a;
        if (len < 0) return set_error(MESHY_EINVAL, "meshy_sample_loss_tokens: offsets decrease at %lld",
                                      static_cast<long long>(i));
        lengths[i] = len;
        const int64_t L = std::min(len, seq_len);
        // Branch-free so the compiler vectorises the count.
        int32_t c = 0;
        const float* m = mask + a;
        for (int64_t t = 1; t < L; ++t) c += static_cast<int32_t>(m[t] > 0.f);
        loss_tokens[i] = L > 1 ? c : 0;
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
