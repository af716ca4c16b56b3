// Counter-based normal variates in fp32 that come out bit-identical on the
// device and the host: a splitmix64 hash of (seed, pair index) gives two
// 32-bit uniforms, and a Box-Muller transform (Box & Muller 1958) turns them
// into two independent N(0, 1) values:
//     u1 = n / 2^32, n = lo32(h) + 1 in [1, 2^32]
//     a  = hi32(h), theta = 2 pi a / 2^32
//     r  = sqrt(-2 ln u1),  (z0, z1) = (r cos theta, r sin theta)
// Every function here uses only fp32 adds, multiplies and fused
// multiply-adds (each correctly rounded, the same on both sides), integer
// operations and exact int-to-float conversions; no library log, sqrt,
// sin, cos or divide is called.  The file is compiled with contraction off
// (-ffp-contract=off and the pragma below), so no add and multiply are fused
// behind the code's back on either side.
//   ln:   u1 = 2^e * m with m in [sqrt(1/2), sqrt 2] (from the 24 leading
//         bits of n, or of 2^32 - n when u1 >= 1/2, so that u1 near 1 keeps
//         its precision); ln m = 2 atanh(s), s = (m - 1) / (m + 1),
//         |s| <= 0.1716, by its Taylor series to s^9 (truncation < 7e-10);
//         e ln 2 in two parts (Cody & Waite 1980) so e * ln2_hi is exact.
//   1/d:  a linear start on [1.70, 2.42] and three Newton steps
//         r <- r + r (1 - d r) (start error < 3 %, then < 1e-12).
//   sqrt: 1/sqrt(x) from the exponent-halving integer start (Lomont 2003,
//         "Fast inverse square root"), three Newton steps, then one
//         Newton correction of x * (1/sqrt(x)).
//   sin, cos: theta's octant from the top 3 bits of a, the angle within it
//         (mirrored in odd octants) in [0, pi/4] from the next 24 bits, the
//         Taylor series of sin to x^9 and cos to x^10 (truncation < 2e-9),
//         then the octant's swap and signs.
// The header also builds with a plain C++ compiler (MESHY_HD empty), which is
// how the CPU tests check each routine against float64.
#pragma once

#include <cmath>
#include <cstdint>

#if defined(__HIPCC__) || defined(__HIP__)
#define MESHY_HD __host__ __device__ __forceinline__
#else
#define MESHY_HD inline
#endif

#pragma STDC FP_CONTRACT OFF

namespace meshy {
namespace synth {

MESHY_HD uint64_t mix64(uint64_t x) {  // splitmix64's finaliser (Steele, Lea, Flood 2014)
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

MESHY_HD float fma32(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
MESHY_HD float bits_to_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
MESHY_HD uint32_t f32_to_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

constexpr float kSqrt2 = 1.41421356f;
constexpr float kLn2Hi = 0.693145751953125f;    // 0x3f317200: e * kLn2Hi is exact for |e| < 2^12
constexpr float kLn2Lo = 1.42860682e-06f;       // ln 2 - kLn2Hi
constexpr float kPi4Over2p24 = 0.785398163397448310f * 0x1p-24f;  // (pi / 4) / 2^24, an exact scaling

// 1 / d for d in [1.70, 2.42].
MESHY_HD float recip_1p7_2p42(float d) {
    float r = fma32(d, -0.2427f, 1.0001f);
    for (int i = 0; i < 3; ++i) r = fma32(r, fma32(-d, r, 1.0f), r);
    return r;
}

// 2 (k ln 2 - ln(1 + f)) for f in [sqrt(1/2) - 1, sqrt 2 - 1] and an
// integer k in [0, 32]; ln(1 + f) = 2 atanh(s), s = f / (2 + f).
MESHY_HD float two_k_ln2_minus_ln1p(int k, float f) {
    const float s = f * recip_1p7_2p42(2.0f + f);
    const float s2 = s * s;
    float p = fma32(s2, 1.0f / 9.0f, 1.0f / 7.0f);
    p = fma32(s2, p, 1.0f / 5.0f);
    p = fma32(s2, p, 1.0f / 3.0f);
    p = fma32(s2, p, 1.0f);
    const float ln1p = 2.0f * (s * p);
    const float kf = static_cast<float>(k);
    float q = fma32(kf, kLn2Hi, -ln1p);
    q = fma32(kf, kLn2Lo, q);
    return 2.0f * q;
}

// The 24 leading bits of v (1 <= v < 2^40) as a float, scaled by 2^-32
// exactly: v 2^-32 with its lower bits dropped.
MESHY_HD float leading24_times_2m32(uint64_t v, int& e) {
    e = 63 - __builtin_clzll(v);                                                  // floor(log2 v)
    const uint32_t m24 = static_cast<uint32_t>((v << (63 - e)) >> 40);
    return static_cast<float>(m24) * bits_to_f32(static_cast<uint32_t>(127 + e - 23 - 32) << 23);
}

// -2 ln(n / 2^32) for n in [1, 2^32]; 0 at n = 2^32, 44.36 at n = 1.
//   n < 2^31: n = 2^e m, m in [sqrt(1/2), sqrt 2] from n's 24 leading bits;
//             the result is 2 ((32 - e) ln 2 - ln m).
//   n >= 2^31: u = 1 - d with d = (2^32 - n) / 2^32 in [0, 1/2], exact up to
//             d's own 24 leading bits, so a u near 1 keeps its precision:
//             ln u = ln(1 - d) directly for d <= 1 - sqrt(1/2), else
//             ln(2 (1 - d)) - ln 2.
MESHY_HD float neg2_ln_unit(uint64_t n) {
    if (n < (1ull << 31)) {
        int e;
        float m = leading24_times_2m32(n, e) * bits_to_f32(static_cast<uint32_t>(127 + 32 - e) << 23);  // [1, 2), exact
        if (m > kSqrt2) {
            m *= 0.5f;                                                             // exact
            e += 1;
        }
        return two_k_ln2_minus_ln1p(32 - e, m - 1.0f);                             // m - 1 exact (Sterbenz)
    }
    const uint64_t c = (1ull << 32) - n;
    if (c == 0) return 0.0f;
    int e;
    const float d = leading24_times_2m32(c, e);                                    // (0, 1/2]
    if (d <= 0.29289322f) return two_k_ln2_minus_ln1p(0, -d);
    const float m = 1.0f - d;                                                      // [1/2, sqrt(1/2))
    return two_k_ln2_minus_ln1p(1, 2.0f * m - 1.0f);                               // 2m - 1 exact
}

// sqrt(x) for finite x >= 0.
MESHY_HD float sqrt32(float x) {
    if (!(x > 0.0f)) return 0.0f;
    float y = bits_to_f32(0x5F375A86u - (f32_to_bits(x) >> 1));               // ~1/sqrt(x), within 3.5 %
    const float h = 0.5f * x;
    for (int i = 0; i < 3; ++i) y = y * fma32(-h, y * y, 1.5f);
    const float r = x * y;
    return fma32(0.5f * y, fma32(-r, r, x), r);
}

// (cos, sin) of 2 pi a / 2^32.
MESHY_HD void cos_sin_turn(uint32_t a, float& c_out, float& s_out) {
    const uint32_t o = a >> 29;                                                // octant
    uint32_t b = a & 0x1FFFFFFFu;
    if (o & 1u) b = 0x20000000u - b;                                           // mirrored: angle from the octant's end
    const float x = static_cast<float>(b >> 5) * kPi4Over2p24;                // [0, pi/4]
    const float x2 = x * x;
    float ps = fma32(x2, 1.0f / 362880.0f, -1.0f / 5040.0f);
    ps = fma32(x2, ps, 1.0f / 120.0f);
    ps = fma32(x2, ps, -1.0f / 6.0f);
    const float sn = fma32(x * x2, ps, x);
    float pc = fma32(x2, -1.0f / 3628800.0f, 1.0f / 40320.0f);
    pc = fma32(x2, pc, -1.0f / 720.0f);
    pc = fma32(x2, pc, 1.0f / 24.0f);
    pc = fma32(x2, pc, -0.5f);
    const float cs = fma32(x2, pc, 1.0f);
    // theta = o pi/4 + x (even o) or (o + 1) pi/4 - x (odd o).
    const bool swap = ((o + 1u) >> 1) & 1u;                                   // octants 1, 2, 5, 6
    const bool neg_c = ((o + 2u) >> 2) & 1u;                                  // octants 2..5
    const bool neg_s = (o >> 2) & 1u;                                         // octants 4..7
    const float c = swap ? sn : cs;
    const float s = swap ? cs : sn;
    c_out = neg_c ? -c : c;
    s_out = neg_s ? -s : s;
}

// The pair of N(0, scale^2) values of hash h: scale * (r cos theta, r sin theta).
MESHY_HD void normal_pair(uint64_t h, float scale, float& z0, float& z1) {
    const uint64_t n = (h & 0xFFFFFFFFull) + 1u;
    const float r = sqrt32(neg2_ln_unit(n)) * scale;
    float c, s;
    cos_sin_turn(static_cast<uint32_t>(h >> 32), c, s);
    z0 = r * c;
    z1 = r * s;
}

// fp32 -> bf16, round to nearest even (finite inputs).
MESHY_HD uint16_t bf16_rne(float x) {
    uint32_t u = f32_to_bits(x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Elements 2p and 2p + 1 of a fill with the given mixed seed.
MESHY_HD void normal_bf16_pair(uint64_t seed_mixed, uint64_t p, float scale, uint16_t& e0, uint16_t& e1) {
    float z0, z1;
    normal_pair(mix64(seed_mixed ^ p), scale, z0, z1);
    e0 = bf16_rne(z0);
    e1 = bf16_rne(z1);
}

}  // namespace synth
}  // namespace meshy
