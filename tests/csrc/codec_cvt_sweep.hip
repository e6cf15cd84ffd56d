// GPU sweep of the two gfx950 packed conversions the codec kernels rely on
// (si_codec_math.h), over every 32-bit float pattern:
//   counts[0]: insert_q<0>(f, 8, 0) != clamp(rne(f), 0, 255), NaN -> 0
//              (v_cvt_pk_u8_f32 as the int8 quantiser uses it);
//   counts[1]: insert_q<0>(f, 4, 0) != clamp(rne(f), 0, 15), NaN -> 0, over
//              every pattern but the signalling NaNs: the quantiser's operand
//              is an FMA result (div_rn), and IEEE arithmetic never returns a
//              signalling NaN (v_med3_f32, the int4 clamp, does not quieten
//              one to 0);
//   counts[2]: pack_bf16x2(f, f) != f32_to_bf16(f) in both halves, f not NaN
//              (v_cvt_pk_bf16_f32 against the integer RNE formula);
//   counts[3]: patterns visited (2^32).
// The references use no conversion instruction: rounding to nearest even is
// done on the integer bit pattern.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "si_codec_math.h"

namespace {

// clamp(rne(f), 0, qmax) for non-NaN f, from the bit pattern.
__device__ uint32_t ref_q(uint32_t u, uint32_t qmax)
{
    const uint32_t mag = u & 0x7fffffffu;
    if (mag > 0x7f800000u) return 0u;        // NaN
    if (u >> 31) return 0u;                  // negative (or -0): clamps to 0
    const int e = int(mag >> 23) - 127;      // f = 1.m * 2^e
    if (e < -1) return 0u;                   // f < 0.5
    if (e >= 9) return qmax;                 // f >= 512
    const uint64_t m = (mag & 0x7fffffu) | 0x800000u;  // f = m * 2^(e-23)
    const int sh = 23 - e;                   // 15 .. 24
    const uint64_t ip = m >> sh, rem = m & ((uint64_t(1) << sh) - 1), half = uint64_t(1) << (sh - 1);
    uint64_t r = ip + ((rem > half || (rem == half && (ip & 1))) ? 1 : 0);
    return r > qmax ? qmax : uint32_t(r);
}

__global__ void sweep(unsigned long long* counts)
{
    unsigned long long bad8 = 0, bad4 = 0, badbf = 0, seen = 0;
    const uint64_t nthreads = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < (uint64_t(1) << 32); i += nthreads) {
        const uint32_t u = uint32_t(i);
        const float f = si::bits_f32(u);
        ++seen;
        if ((si::insert_q<0>(f, 8, 0u) & 0xffu) != ref_q(u, 255)) ++bad8;
        const bool snan = (u & 0x7fffffffu) > 0x7f800000u && !(u & 0x00400000u);
        if (!snan && (si::insert_q<0>(f, 4, 0u) & 0xffu) != ref_q(u, 15)) ++bad4;
        if ((u & 0x7fffffffu) <= 0x7f800000u) {
            const uint32_t p = si::pack_bf16x2(f, f), w = si::f32_to_bf16(f);
            if ((p & 0xffffu) != w || (p >> 16) != w) ++badbf;
        }
    }
    atomicAdd(counts + 0, bad8);
    atomicAdd(counts + 1, bad4);
    atomicAdd(counts + 2, badbf);
    atomicAdd(counts + 3, seen);
}

}  // namespace

// counts: device array of 4 zeroed u64.  Returns 0 when queued.
extern "C" int si_selftest_cvt_sweep(hipStream_t stream, unsigned long long* counts)
{
    if (!counts) return -1;
    hipLaunchKernelGGL(sweep, dim3(8192), dim3(256), 0, stream, counts);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
