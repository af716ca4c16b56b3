// Planner (meshy_plan_build) under the sanitizers: 3000 random batches and
// configurations, valid and invalid (dp 1/2/4, up to 156 samples, empty and
// one-token samples, samples over the budget, both layouts, budgets and row
// caps on and off), with the tables sized as include/meshy_amd.h documents.
// Built from meshy_amd/csrc/plan.cpp by tests/test_native_host_cpu.py.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "../../meshy_amd/csrc/host_common.h"

namespace meshy {
int set_error(int code, const char*, ...) { return code; }
void clear_error() {}
}  // namespace meshy

int main() {
    unsigned s = 7;
    auto rnd = [&s](unsigned m) { s = s * 1664525u + 1013904223u; return (s >> 8) % m; };
    int built = 0, rejected = 0;
    for (int it = 0; it < 3000; ++it) {
        const int64_t dp = int64_t{1} << rnd(3);
        const int64_t n = dp * static_cast<int64_t>(rnd(40));
        const int64_t align = int64_t{1} << rnd(12);
        const int64_t seq_len = align * (1 + rnd(16));
        std::vector<int64_t> len(n), loss(n);
        for (int64_t i = 0; i < n; ++i) {
            len[i] = rnd(5) == 0 ? rnd(3) : rnd(static_cast<unsigned>(seq_len) * 2 + 1);
            loss[i] = len[i] > 1 ? rnd(static_cast<unsigned>(len[i])) : 0;
        }
        meshy_planner_cfg cfg{};
        cfg.layout = static_cast<int32_t>(rnd(2));
        cfg.mini_batch_size = 1 + rnd(12);
        cfg.seq_len = seq_len;
        cfg.align = align;
        cfg.max_tokens_per_micro = rnd(3) ? seq_len * (1 + rnd(4)) : 0;
        cfg.micro_batch_size = rnd(2) ? 1 + rnd(6) : 0;
        const int64_t n_local = n / dp;
        const int64_t n_mini = (n_local + cfg.mini_batch_size - 1) / cfg.mini_batch_size;
        std::vector<int32_t> local(dp * n_local + 1), mini_micro(n_mini + 1), doc_start(dp * (n_local + 1) + 1),
            doc_sample(dp * n_local + 1);
        std::vector<int64_t> docs_g(n_mini + 1), tokens_g(n_mini + 1), per_rank(n_mini * dp + 1),
            seq(dp * n_local + 1), doc_len(dp * n_local + 1);
        meshy_plan_out out{local.data(), mini_micro.data(), docs_g.data(), tokens_g.data(), per_rank.data(),
                           seq.data(), doc_start.data(), doc_sample.data(), doc_len.data(), 0, 0};
        if (meshy_plan_build(len.data(), loss.data(), n, dp, &cfg, &out) == MESHY_OK) {
            ++built;
            if (out.n_micro_total > n_local && n_local > 0) {
                std::printf("rank has %d micros for %lld samples\n", out.n_micro_total,
                            static_cast<long long>(n_local));
                return 1;
            }
        } else {
            ++rejected;
        }
    }
    std::printf("plan harness: %d built, %d rejected\n", built, rejected);
    return built == 0;
}
