// CPU check of the codec quantiser's division (si_codec_math.h): for normal
// scales s (with 1/s normal) and numerators a >= 0 with a/s < 2^23,
//   * recip_refine(s, y0) returns RN(1/s) for every estimate y0 within 2 ulp
//     of 1/s (the device's v_rcp_f32 estimate is within 1 ulp);
//   * div_rn(a, s, RN(1/s)) equals the IEEE quotient RN(a/s) bit for bit when
//     a is 0 or a >= 2^-100 (the residual a - q*s is then exact in fp32);
//   * for 0 < a < 2^-100 (subnormal or tiny normal numerators, whose FMA
//     residual may round) both quotients are below 2^-60 at the codec's
//     scales (s >= 1e-12) and round to the same integer (0), which is all the
//     quantiser keeps.
// Cases: random (s, a), quotients next to the rounding ties k + 0.5 (where a
// division formed as a * RN(1/s) goes wrong) and next to integers,
// numerators near the bottom of the normal range, and the codec's own scales
// (hi - lo) / qmax of bf16 values for qmax = 15, 255.
// Built for the host only (hipcc --cuda-host-only); prints "cases N bad M".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>

#include "si_codec_math.h"

using si::bits_f32;
using si::f32_bits;

static uint64_t g_cases = 0, g_bad = 0, g_naive_diff = 0, g_tiny = 0;

static void check(float a, float s)
{
    if (!(s > 0) || !std::isnormal(s) || !std::isnormal(1.0f / s) || a < 0) return;
    const float want = a / s;
    if (!(want < 8388608.0f)) return;
    const float r = 1.0f / s;
    for (int d = -2; d <= 2; ++d) {
        const float y0 = bits_f32(f32_bits(r) + uint32_t(d));
        const float y = si::recip_refine(s, y0);
        const float got = si::div_rn(a, s, y);
        ++g_cases;
        const bool tiny = a != 0.0f && a < 0x1p-100f;
        g_tiny += tiny ? 1 : 0;
        // tiny numerators: only the codec's scales are in scope
        if (tiny && s < 1e-12f) continue;
        const bool same = tiny ? (got < 0x1p-60f && want < 0x1p-60f && std::nearbyint(got) == std::nearbyint(want))
                               : f32_bits(got) == f32_bits(want);
        if (f32_bits(y) != f32_bits(r) || !same) {
            if (g_bad < 10)
                std::printf("mismatch a=%a s=%a y0=%a: recip %a (want %a) div %a (want %a)\n", a, s, y0, y, r, got,
                            want);
            ++g_bad;
        }
    }
    if (f32_bits(a * r) != f32_bits(want)) ++g_naive_diff;
}

int main()
{
    std::mt19937_64 rng(20261202);
    std::uniform_real_distribution<float> expo(-40.0f, 40.0f), unit(0.0f, 1.0f);
    // random scales and numerators
    for (int i = 0; i < 2000000; ++i) {
        const float s = std::ldexp(1.0f + unit(rng), int(expo(rng)));
        const float q = unit(rng) * 300.0f;
        check(q * s, s);
    }
    // quotients near k + 0.5 and near integers: a = (k + 0.5) * s nudged by a few ulp
    for (int i = 0; i < 2000000; ++i) {
        const float s = std::ldexp(1.0f + unit(rng), int(expo(rng)));
        const int k = int(unit(rng) * 256.0f);
        const float base = (i & 1) ? (float(k) + 0.5f) * s : float(k) * s;
        for (int d = -3; d <= 3; ++d) check(bits_f32(f32_bits(base) + uint32_t(d)), s);
    }
    // numerators at the bottom of the normal range and subnormal ones
    for (int i = 0; i < 500000; ++i) {
        const float s = std::ldexp(1.0f + unit(rng), int(expo(rng)));
        const float a = (i & 1) ? std::ldexp(1.0f + unit(rng), -126 + int(unit(rng) * 8.0f))
                                : bits_f32(uint32_t(unit(rng) * 8388607.0f) + 1u);
        check(a, s);
    }
    // the codec's scales: (hi - lo) / qmax of bf16-valued hi, lo
    for (int i = 0; i < 1000000; ++i) {
        const float lo = bits_f32(f32_bits(std::ldexp(unit(rng) - 0.5f, int(expo(rng) / 4))) & 0xffff0000u);
        const float hi = bits_f32(f32_bits(lo + std::ldexp(unit(rng), int(expo(rng) / 4))) & 0xffff0000u);
        for (float qmax : {15.0f, 255.0f}) {
            float s = (hi - lo) / qmax;
            if (s < 1e-12f) s = 1e-12f;
            const float x = bits_f32(f32_bits(lo + unit(rng) * (hi - lo)) & 0xffff0000u);
            check(x - lo, s);
        }
    }
    std::printf("cases %llu bad %llu naive_differs %llu tiny_numerators %llu\n",
                (unsigned long long)g_cases, (unsigned long long)g_bad, (unsigned long long)g_naive_diff,
                (unsigned long long)g_tiny);
    return g_bad ? 1 : 0;
}
