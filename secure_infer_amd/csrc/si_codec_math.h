// Rounding helpers of the KV transport codec kernels (si_codec.hip).  The
// float semantics follow the reference's torch ops one rounding at a time
// (transport_codec.py:22-42, optimized_decode.py:5-26).  The host-callable
// ones are also compiled into the CPU check of the division
// (tests/csrc/codec_div_check.hip), and the device conversions into the
// GPU sweep over every float bit pattern (tests/csrc/codec_cvt_sweep.hip),
// so both test exactly the code the kernels run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

__host__ __device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// bf16 round-to-nearest-even of a float; every NaN becomes 0x7fc0 (torch's
// float -> bfloat16 conversion).
__host__ __device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// RN(1/s) for a normal s from an estimate y0 within a few ulp of 1/s: two
// Newton steps, then the neighbour with the smallest exact residual
// |1 - s*y| (one FMA each).  The device passes v_rcp_f32's estimate.
__host__ __device__ __forceinline__ float recip_refine(float s, float y0)
{
    float y = y0;
    y = fmaf(fmaf(-s, y, 1.0f), y, y);
    y = fmaf(fmaf(-s, y, 1.0f), y, y);
    const float ylo = bits_f32(f32_bits(y) - 1u);
    const float yhi = bits_f32(f32_bits(y) + 1u);
    const float e = fabsf(fmaf(-s, y, 1.0f));
    const float elo = fabsf(fmaf(-s, ylo, 1.0f));
    const float ehi = fabsf(fmaf(-s, yhi, 1.0f));
    if (elo < e) return ylo;
    if (ehi < e) return yhi;
    return y;
}

// RN(a/s) given y = RN(1/s) (Markstein: q within 1 ulp of a/s, exact FMA
// residual r = a - q*s, q + r*y rounds correctly); a >= 0, a/s < 2^23.
// Build with -ffp-contract=off: a*y must round on its own.
__host__ __device__ __forceinline__ float div_rn(float a, float s, float y)
{
    const float q = a * y;
    return fmaf(fmaf(-q, s, a), y, q);
}

__device__ __forceinline__ float recip_rn(float s) { return recip_refine(s, __builtin_amdgcn_rcpf(s)); }

// Quantised value v (already RN((x - lo) / s)) inserted as byte K of acc:
// v_cvt_pk_u8_f32 rounds to nearest even, saturates to [0, 255] and sends
// NaN to 0 (checked on every float bit pattern against
// clamp(rne(f), 0, 255)), so int8 needs no clamp of its own; int4 clamps to
// [0, 15] first (the clamp commutes with rounding: integer bounds).
template <int K>
__device__ __forceinline__ uint32_t insert_q(float v, uint32_t bits, uint32_t acc)
{
    if (bits != 8) v = __builtin_amdgcn_fmed3f(v, 0.0f, 15.0f);
    return __builtin_amdgcn_cvt_pk_u8_f32(v, K, acc);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats as packed bf16 with v_cvt_pk_bf16_f32: round to nearest even,
// identical to f32_to_bf16 for every non-NaN float (checked on every bit
// pattern); a NaN keeps its sign and payload, so callers route NaN to
// f32_to_bf16.
__device__ __forceinline__ uint32_t pack_bf16x2(float v0, float v1)
{
    f32x2 v;
    v.x = v0;
    v.y = v1;
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

}  // namespace si
