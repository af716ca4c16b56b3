// Evaluates the fp32 routines of synth_math.h over an input file, for the CPU
// tests that compare them with float64 (built with g++, no HIP).
//   synth_math_harness ln    in.u64 out.f32     -2 ln(n / 2^32)
//   synth_math_harness sqrt  in.f32 out.f32     sqrt(x)
//   synth_math_harness turn  in.u32 out.f32x2   (cos, sin)(2 pi a / 2^32)
//   synth_math_harness pair  in.u64 out.f32x2   the N(0, 1) pair of hash h
//   synth_math_harness bf16  in.u64 out.u16x2   bf16 pair p of seed 1, scale 2
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "synth_math.h"

template <class T>
static std::vector<T> read_all(const char* path) {
    std::vector<T> v;
    FILE* f = std::fopen(path, "rb");
    if (!f) std::exit(2);
    T x;
    while (std::fread(&x, sizeof(T), 1, f) == 1) v.push_back(x);
    std::fclose(f);
    return v;
}

template <class T>
static void write_all(const char* path, const std::vector<T>& v) {
    FILE* f = std::fopen(path, "wb");
    if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) std::exit(3);
    std::fclose(f);
}

int main(int argc, char** argv) {
    using namespace meshy::synth;
    if (argc != 4) return 1;
    const char* mode = argv[1];
    if (!std::strcmp(mode, "ln")) {
        std::vector<float> out;
        for (uint64_t n : read_all<uint64_t>(argv[2])) out.push_back(neg2_ln_unit(n));
        write_all(argv[3], out);
    } else if (!std::strcmp(mode, "sqrt")) {
        std::vector<float> out;
        for (float x : read_all<float>(argv[2])) out.push_back(sqrt32(x));
        write_all(argv[3], out);
    } else if (!std::strcmp(mode, "turn")) {
        std::vector<float> out;
        for (uint32_t a : read_all<uint32_t>(argv[2])) {
            float c, s;
            cos_sin_turn(a, c, s);
            out.push_back(c);
            out.push_back(s);
        }
        write_all(argv[3], out);
    } else if (!std::strcmp(mode, "pair")) {
        std::vector<float> out;
        for (uint64_t h : read_all<uint64_t>(argv[2])) {
            float z0, z1;
            normal_pair(h, 1.0f, z0, z1);
            out.push_back(z0);
            out.push_back(z1);
        }
        write_all(argv[3], out);
    } else if (!std::strcmp(mode, "bf16")) {
        std::vector<uint16_t> out;
        const uint64_t sm = mix64(1);
        for (uint64_t p : read_all<uint64_t>(argv[2])) {
            uint16_t e0, e1;
            normal_bf16_pair(sm, p, 2.0f, e0, e1);
            out.push_back(e0);
            out.push_back(e1);
        }
        write_all(argv[3], out);
    } else {
        return 1;
    }
    return 0;
}
