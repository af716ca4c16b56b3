// Host gather (meshy_host_gather) under the sanitizers: four threads call it at
// once, 60 gathers each, with 1 to 200 pieces of up to 40000 bytes, thread caps
// 0, 4 and 8; every output is compared with the pieces.  Built from
// meshy_amd/csrc/hostio.cpp by tests/test_native_host_cpu.py.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../meshy_amd/csrc/host_common.h"

namespace meshy {
int set_error(int code, const char*, ...) { return code; }
void clear_error() {}
}  // namespace meshy

int main() {
    constexpr int kCallers = 4, kJobs = 60;
    std::vector<int> bad(kCallers, 0);
    std::vector<std::thread> callers;
    for (int c = 0; c < kCallers; ++c) {
        callers.emplace_back([c, &bad] {
            unsigned s = 1234u + c;
            auto rnd = [&s](unsigned m) { s = s * 1664525u + 1013904223u; return (s >> 8) % m; };
            for (int j = 0; j < kJobs; ++j) {
                const int n = 1 + static_cast<int>(rnd(200));
                std::vector<std::vector<char>> parts(n);
                std::vector<const void*> ptr(n);
                std::vector<int64_t> size(n);
                int64_t total = 0;
                for (int i = 0; i < n; ++i) {
                    parts[i].resize(rnd(40000));
                    for (size_t b = 0; b < parts[i].size(); ++b) parts[i][b] = static_cast<char>((i * 31 + b + c) & 0x7f);
                    ptr[i] = parts[i].data();
                    size[i] = static_cast<int64_t>(parts[i].size());
                    total += size[i];
                }
                std::vector<char> out(total + 1);
                if (meshy_host_gather(ptr.data(), size.data(), n, out.data(), (j % 3) * 4) != MESHY_OK) {
                    ++bad[c];
                    continue;
                }
                int64_t o = 0;
                for (int i = 0; i < n; ++i) {
                    if (size[i] && std::memcmp(out.data() + o, parts[i].data(), size[i]) != 0) ++bad[c];
                    o += size[i];
                }
            }
        });
    }
    for (auto& t : callers) t.join();
    int total_bad = 0;
    for (int b : bad) total_bad += b;
    std::printf("gather harness: %d bad gathers\n", total_bad);
    return total_bad != 0;
}
