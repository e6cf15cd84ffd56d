// KV transport codec kernels (int8 / int4, asymmetric min/max, group 64).
//
// Packet of one record (one 128-token block of one kind, [128, h, d] bf16):
//   [q: 128*h*d*bits/8][scale f32: 2*h*d][low f32: 2*h*d][int32 {1, layer,
//   kind, bits}][zero pad to 16]
// K (kind 0) groups 64 tokens per (h, d): params (2, h, d).  V (kind 1) groups
// 64 dims per (t, h): params (128, h, d/64).  int4 packs element 2i in the
// low nibble.  (transport_codec.py:22-42, optimized_decode.py:5-26.)
//
// Float semantics follow the reference's torch ops one rounding at a time:
// decode v = fl(fl(q*scale) + low) then bf16 round-to-nearest-even; encode
// scale = max(fl((hi-lo)/(2^bits-1)), 1e-12f), q = clamp(rne(fl(fl(x-lo)/scale))).
#include "si_kernels.h"

namespace si {

__device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h)
{
    return __uint_as_float(h << 16);
}

// One thread -> 8 consecutive elements (16 B of bf16 output).
__global__ __launch_bounds__(256) void dequant_scatter_kernel(CodecBatch b, uint32_t groups_per_rec)
{
    const uint32_t r = blockIdx.x / groups_per_rec;
    const uint32_t g = (blockIdx.x % groups_per_rec) * 256u + threadIdx.x;
    const uint32_t hd = b.heads * b.dim;
    const uint32_t total = 128u * hd;
    const uint32_t e0 = g * 8u;
    if (e0 >= total) return;
    const uint32_t kind = r < b.n_k ? 0u : 1u;
    const uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    const float* scale = reinterpret_cast<const float*>(pkt + b.qbytes);
    const float* low = reinterpret_cast<const float*>(pkt + b.qbytes + b.sbytes);
    const uint32_t t = e0 / hd;
    const uint32_t rem = e0 % hd;
    const uint32_t hh = rem / b.dim;
    const uint32_t dd = rem % b.dim;

    float q[8];
    if (b.bits == 8) {
        const uint2 w = *reinterpret_cast<const uint2*>(pkt + e0);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            q[k] = float((w.x >> (8 * k)) & 0xffu);
            q[4 + k] = float((w.y >> (8 * k)) & 0xffu);
        }
    } else {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(pkt + e0 / 2);
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = float((w >> (4 * k)) & 0xfu);
    }
    float s[8], o[8];
    if (kind == 0) {
        const uint32_t p = (t / 64u) * hd + rem;
#pragma unroll
        for (int k = 0; k < 8; ++k) { s[k] = scale[p + k]; o[k] = low[p + k]; }
    } else {
        const uint32_t p = (t * b.heads + hh) * (b.dim / 64u) + dd / 64u;
        const float sv = scale[p], ov = low[p];
#pragma unroll
        for (int k = 0; k < 8; ++k) { s[k] = sv; o[k] = ov; }
    }
    uint32_t out[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float v0 = __fadd_rn(__fmul_rn(q[2 * k], s[2 * k]), o[2 * k]);
        const float v1 = __fadd_rn(__fmul_rn(q[2 * k + 1], s[2 * k + 1]), o[2 * k + 1]);
        out[k] = f32_to_bf16(v0) | (f32_to_bf16(v1) << 16);
    }
    const int64_t sid = b.slots[r];
    if (sid < 0 || sid >= b.nslots) return;
    uint8_t* slot = b.cache[kind] + uint64_t(sid) * b.slot_bytes;
    *reinterpret_cast<uint4*>(slot + uint64_t(e0) * 2u) = make_uint4(out[0], out[1], out[2], out[3]);
}

__device__ __forceinline__ float quant_scale(float lo, float hi, float qmax)
{
    const float s = __fdiv_rn(__fsub_rn(hi, lo), qmax);
    return s < 1e-12f ? 1e-12f : s;
}

__device__ __forceinline__ uint32_t quant_one(float x, float lo, float s, float qmax)
{
    float q = rintf(__fdiv_rn(__fsub_rn(x, lo), s));
    q = q < 0.f ? 0.f : q;
    q = q > qmax ? qmax : q;
    return uint32_t(q);
}

// K: one thread per (token group, head, column pair).
__global__ __launch_bounds__(256) void quant_k_kernel(CodecBatch b, uint32_t rec0, uint32_t blocks_per_rec)
{
    const uint32_t r = rec0 + blockIdx.x / blocks_per_rec;
    const uint32_t idx = (blockIdx.x % blocks_per_rec) * 256u + threadIdx.x;
    const uint32_t hd = b.heads * b.dim;
    if (idx >= hd) return;  // 2 groups * hd/2 column pairs
    const uint32_t grp = idx / (hd / 2u);
    const uint32_t col = (idx % (hd / 2u)) * 2u;
    const float qmax = float((1u << b.bits) - 1u);
    const int64_t sid = b.slots[r];
    if (sid < 0 || sid >= b.nslots) return;
    const uint8_t* slot = b.cache[0] + uint64_t(sid) * b.slot_bytes;
    uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    float lo0 = INFINITY, lo1 = INFINITY, hi0 = -INFINITY, hi1 = -INFINITY;
    for (uint32_t tt = 0; tt < 64u; ++tt) {
        const uint32_t t = grp * 64u + tt;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(slot + (uint64_t(t) * hd + col) * 2u);
        const float x0 = bf16_to_f32(w & 0xffffu), x1 = bf16_to_f32(w >> 16);
        lo0 = fminf(lo0, x0); hi0 = fmaxf(hi0, x0);
        lo1 = fminf(lo1, x1); hi1 = fmaxf(hi1, x1);
    }
    const float s0 = quant_scale(lo0, hi0, qmax), s1 = quant_scale(lo1, hi1, qmax);
    const uint32_t p = grp * hd + col;
    float* scale = reinterpret_cast<float*>(pkt + b.qbytes);
    float* low = reinterpret_cast<float*>(pkt + b.qbytes + b.sbytes);
    scale[p] = s0; scale[p + 1] = s1;
    low[p] = lo0; low[p + 1] = lo1;
    for (uint32_t tt = 0; tt < 64u; ++tt) {
        const uint32_t t = grp * 64u + tt;
        const uint64_t e = uint64_t(t) * hd + col;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(slot + e * 2u);
        const uint32_t q0 = quant_one(bf16_to_f32(w & 0xffffu), lo0, s0, qmax);
        const uint32_t q1 = quant_one(bf16_to_f32(w >> 16), lo1, s1, qmax);
        if (b.bits == 8)
            *reinterpret_cast<uint16_t*>(pkt + e) = uint16_t(q0 | (q1 << 8));
        else
            pkt[e / 2] = uint8_t(q0 | (q1 << 4));
    }
}

// V: one thread per (token, head, dim group of 64).
__global__ __launch_bounds__(256) void quant_v_kernel(CodecBatch b, uint32_t rec0, uint32_t blocks_per_rec)
{
    const uint32_t r = rec0 + blockIdx.x / blocks_per_rec;
    const uint32_t idx = (blockIdx.x % blocks_per_rec) * 256u + threadIdx.x;
    const uint32_t ng = b.dim / 64u;
    const uint32_t hd = b.heads * b.dim;
    if (idx >= 128u * b.heads * ng) return;
    const uint32_t t = idx / (b.heads * ng);
    const uint32_t hh = (idx / ng) % b.heads;
    const uint32_t dg = idx % ng;
    const float qmax = float((1u << b.bits) - 1u);
    const int64_t sid = b.slots[r];
    if (sid < 0 || sid >= b.nslots) return;
    const uint8_t* slot = b.cache[1] + uint64_t(sid) * b.slot_bytes;
    uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    const uint64_t e0 = uint64_t(t) * hd + uint64_t(hh) * b.dim + dg * 64u;
    const uint4* src = reinterpret_cast<const uint4*>(slot + e0 * 2u);
    uint32_t raw[32];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint4 v = src[k];
        raw[4 * k] = v.x; raw[4 * k + 1] = v.y; raw[4 * k + 2] = v.z; raw[4 * k + 3] = v.w;
    }
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const float a = bf16_to_f32(raw[k] & 0xffffu), c = bf16_to_f32(raw[k] >> 16);
        lo = fminf(lo, fminf(a, c));
        hi = fmaxf(hi, fmaxf(a, c));
    }
    const float s = quant_scale(lo, hi, qmax);
    const uint32_t p = idx;  // (t, h, dg) row-major == idx
    reinterpret_cast<float*>(pkt + b.qbytes)[p] = s;
    reinterpret_cast<float*>(pkt + b.qbytes + b.sbytes)[p] = lo;
    uint32_t qw[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) qw[k] = 0;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const uint32_t q0 = quant_one(bf16_to_f32(raw[k] & 0xffffu), lo, s, qmax);
        const uint32_t q1 = quant_one(bf16_to_f32(raw[k] >> 16), lo, s, qmax);
        if (b.bits == 8) {
            // elements 2k, 2k+1 -> bytes 2k, 2k+1
            qw[k >> 1] |= (q0 | (q1 << 8)) << (16 * (k & 1));
        } else {
            // byte k = q[2k] | q[2k+1] << 4
            qw[k >> 2] |= (q0 | (q1 << 4)) << (8 * (k & 3));
        }
    }
    if (b.bits == 8) {
        uint4* dst = reinterpret_cast<uint4*>(pkt + e0);
#pragma unroll
        for (int k = 0; k < 4; ++k) dst[k] = make_uint4(qw[4 * k], qw[4 * k + 1], qw[4 * k + 2], qw[4 * k + 3]);
    } else {
        uint4* dst = reinterpret_cast<uint4*>(pkt + e0 / 2);
#pragma unroll
        for (int k = 0; k < 2; ++k) dst[k] = make_uint4(qw[4 * k], qw[4 * k + 1], qw[4 * k + 2], qw[4 * k + 3]);
    }
}

// Header {1, layer, kind, bits} and the zero pad of every packet.
__global__ void packet_tail_kernel(CodecBatch b)
{
    const uint32_t r = blockIdx.x;
    uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    const uint64_t h0 = b.qbytes + 2 * b.sbytes;
    const uint32_t kind = r < b.n_k ? 0u : 1u;
    for (uint64_t i = h0 + threadIdx.x; i < b.width; i += blockDim.x) {
        const uint64_t o = i - h0;
        uint32_t word = 0;
        if (o < 16) {
            const uint32_t f = uint32_t(o / 4);
            word = f == 0 ? 1u : f == 1 ? b.layer : f == 2 ? kind : b.bits;
        }
        pkt[i] = o < 16 ? uint8_t(word >> (8 * (o & 3))) : 0;
    }
}

hipError_t launch_dequant_scatter(hipStream_t stream, const CodecBatch& b)
{
    const uint32_t total8 = 128u * b.heads * b.dim / 8u;
    const uint32_t gpr = (total8 + 255u) / 256u;
    hipLaunchKernelGGL(dequant_scatter_kernel, dim3(b.nrec * gpr), dim3(256), 0, stream, b, gpr);
    return hipGetLastError();
}

hipError_t launch_gather_quant(hipStream_t stream, const CodecBatch& b)
{
    const uint32_t hd = b.heads * b.dim;
    const uint32_t nv = b.nrec - b.n_k;
    if (b.n_k) {
        const uint32_t bpr = (hd + 255u) / 256u;
        hipLaunchKernelGGL(quant_k_kernel, dim3(b.n_k * bpr), dim3(256), 0, stream, b, 0u, bpr);
    }
    if (nv) {
        const uint32_t bpr = (128u * b.heads * (b.dim / 64u) + 255u) / 256u;
        hipLaunchKernelGGL(quant_v_kernel, dim3(nv * bpr), dim3(256), 0, stream, b, b.n_k, bpr);
    }
    hipLaunchKernelGGL(packet_tail_kernel, dim3(b.nrec), dim3(64), 0, stream, b);
    return hipGetLastError();
}

}  // namespace si
