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
// scale = max(fl((hi-lo)/(2^bits-1)), 1e-12f), q = clamp(rne(fl(fl(x-lo)/scale))),
// with fl(a/scale) formed from the correctly rounded reciprocal of the
// group's scale and one FMA correction (bit-identical to IEEE division).
// Non-finite KV follows torch: x.amin / x.amax propagate NaN, so a group with
// a NaN gets NaN scale and low and quantises to 0; an int4 byte whose pair
// holds a NaN quotient is 0 (packed in float, then cast); decoding a NaN
// gives the bf16 NaN 0x7fc0.  The bit patterns of NaN parameters are not
// specified.
#include "si_codec_math.h"
#include "si_clock.h"
#include "si_kernels.h"

namespace si {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t h)
{
    return __uint_as_float(h << 16);
}

// n / d for n < 2^24, d < 2^16 (exact): float estimate, then one correction.
__device__ __forceinline__ uint32_t udiv_small(uint32_t n, uint32_t d)
{
    uint32_t q = uint32_t(__fmul_rn(float(n), __frcp_rn(float(d))));
    if (q * d > n) --q;
    else if ((q + 1u) * d <= n) ++q;
    return q;
}

// Two decoded elements fl(fl(q*s) + o) as packed bf16.  With finite s and o
// no result is NaN (q is a small integer), and v_cvt_pk_bf16_f32 rounds every
// non-NaN float to nearest even exactly like f32_to_bf16 (checked on every
// float bit pattern); a NaN would keep its sign and payload instead of
// becoming 0x7fc0, so non-finite parameters take the scalar conversion.
template <bool kFinite>
__device__ __forceinline__ uint32_t dq2(float q0, float s0, float o0, float q1, float s1, float o1)
{
    const float v0 = __fadd_rn(__fmul_rn(q0, s0), o0);
    const float v1 = __fadd_rn(__fmul_rn(q1, s1), o1);
    if constexpr (kFinite) {
        return pack_bf16x2(v0, v1);
    } else {
        return f32_to_bf16(v0) | (f32_to_bf16(v1) << 16);
    }
}

// 0 for finite x, NaN otherwise (x - x).
__device__ __forceinline__ float nonfinite(float x)
{
    return __fsub_rn(x, x);
}

// One thread -> 16 consecutive columns (h, d) of `tpt` consecutive tokens
// (tpt divides 64) of record r; workgroup x of the record.  A K thread loads
// its 16 (scale, low) pairs once for its tokens (they depend on the column
// and the 64-token group only), so K takes more tokens per thread than V
// (whose pair changes with the token); a V token row of 16 elements shares
// one (t, h, dim-group) pair.  Per token the thread reads 16 (int8) or 8
// (int4) packet bytes and writes 32 bytes of bf16, and a wave covers 1 KiB of
// consecutive packet columns.
__device__ __forceinline__ void dequant_scatter_body(const CodecBatch& b, uint32_t r, uint32_t x, uint32_t tpt)
{
    // An allocation-free call that does not own the GPU's scratch (whose
    // staging this reads) touches nothing; its records are failed closed
    // by the call's finishing kernel.
    if (b.gate && *b.gate == 0u) return;
    const uint32_t hd = b.heads * b.dim;
    const uint32_t nc = hd / 16u;  // column chunks per token
    const uint32_t idx = x * 256u + threadIdx.x;
    if (idx >= (128u / tpt) * nc) return;
    const int64_t sid = b.slots[r];
    if (sid < 0 || sid >= b.nslots) return;
    const uint32_t tg = idx / nc;
    const uint32_t col = (idx - tg * nc) * 16u;
    const uint32_t kind = r < b.n_k ? 0u : 1u;
    const uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    const float* scale = reinterpret_cast<const float*>(pkt + b.qbytes);
    const float* low = reinterpret_cast<const float*>(pkt + b.qbytes + b.sbytes);
    uint8_t* slot = b.cache[kind] + uint64_t(sid) * b.slot_bytes;

    float ks[16], ko[16];
    bool kfin = true;
    if (kind == 0) {
        const uint32_t p = (tg * tpt >> 6) * hd + col;
        const float4* s4 = reinterpret_cast<const float4*>(scale + p);
        const float4* o4 = reinterpret_cast<const float4*>(low + p);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 sv = s4[k], ov = o4[k];
            ks[4 * k] = sv.x; ks[4 * k + 1] = sv.y; ks[4 * k + 2] = sv.z; ks[4 * k + 3] = sv.w;
            ko[4 * k] = ov.x; ko[4 * k + 1] = ov.y; ko[4 * k + 2] = ov.z; ko[4 * k + 3] = ov.w;
        }
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __fadd_rn(acc, __fadd_rn(nonfinite(ks[k]), nonfinite(ko[k])));
        kfin = acc == 0.0f;
    }
    const uint32_t hh = udiv_small(col, b.dim);
    const uint32_t vgroup = hh * (b.dim / 64u) + (col - hh * b.dim) / 64u;
#pragma unroll 2
    for (uint32_t tt = 0; tt < tpt; ++tt) {
        const uint32_t t = tg * tpt + tt;
        const uint32_t e0 = t * hd + col;
        float q[16];
        if (b.bits == 8) {
            const uint4 w = *reinterpret_cast<const uint4*>(pkt + e0);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 16; ++k) q[k] = float((ww[k >> 2] >> (8 * (k & 3))) & 0xffu);
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(pkt + e0 / 2u);
            const uint32_t ww[2] = {w.x, w.y};
#pragma unroll
            for (int k = 0; k < 16; ++k) q[k] = float((ww[k >> 3] >> (4 * (k & 7))) & 0xfu);
        }
        uint32_t out[8];
        if (kind == 0) {
            if (kfin) {
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    out[k] = dq2<true>(q[2 * k], ks[2 * k], ko[2 * k], q[2 * k + 1], ks[2 * k + 1], ko[2 * k + 1]);
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    out[k] = dq2<false>(q[2 * k], ks[2 * k], ko[2 * k], q[2 * k + 1], ks[2 * k + 1], ko[2 * k + 1]);
            }
        } else {
            const uint32_t p = t * (hd / 64u) + vgroup;  // (t, h, dim-group) row-major
            const float sv = scale[p], ov = low[p];
            if (__fadd_rn(nonfinite(sv), nonfinite(ov)) == 0.0f) {
#pragma unroll
                for (int k = 0; k < 8; ++k) out[k] = dq2<true>(q[2 * k], sv, ov, q[2 * k + 1], sv, ov);
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) out[k] = dq2<false>(q[2 * k], sv, ov, q[2 * k + 1], sv, ov);
            }
        }
        // Non-temporal stores: the slots are not read again in this launch,
        // and a kernel that ends with the layer's bf16 output dirty in L2
        // holds the next launch back while that is written back (MI355X,
        // ABBA x 2 on one GPU, layer time: int4 Qwen2.5-7B 24.2 -> 22.7 us,
        // int8 Llama-3-8B 39.3 -> 39.5 us; write-through stores of the two
        // interleaved halves: 32.0 / 56.9 us).
        u32x4* dst = reinterpret_cast<u32x4*>(slot + uint64_t(e0) * 2u);
        const u32x4 v0 = {out[0], out[1], out[2], out[3]}, v1 = {out[4], out[5], out[6], out[7]};
        __builtin_nontemporal_store(v0, dst);
        __builtin_nontemporal_store(v1, dst + 1);
    }
}

// The kx workgroups of each K record (tk tokens per thread), then the vx of
// each V record (tv tokens per thread).
__global__ __launch_bounds__(256) void dequant_scatter_kernel(CodecBatch b, uint32_t kx, uint32_t vx, uint32_t tk,
                                                              uint32_t tv)
{
    clock_stamp(b.clock, 0);
    const uint32_t nkb = kx * b.n_k;
    if (blockIdx.x < nkb) {
        dequant_scatter_body(b, blockIdx.x / kx, blockIdx.x % kx, tk);
    } else {
        const uint32_t v = blockIdx.x - nkb;
        dequant_scatter_body(b, b.n_k + v / vx, v % vx, tv);
    }
    clock_stamp(b.clock, 1);
}

// Another lane's value by a DPP move: 0xb1 swaps lanes 2i / 2i+1, 0x4e swaps
// pairs within a quad, 0x141 mirrors each 8-lane half-row.
template <int kCtrl>
__device__ __forceinline__ float lane_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// x.amin / x.amax semantics (transport_codec.py:30-31): a NaN anywhere in the
// group makes the result NaN; equal zeros order -0 < +0.  v_minimum3_f32 /
// v_maximum3_f32 (IEEE 754-2019 minimum / maximum).
__device__ __forceinline__ float nmin(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float nmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// v[k] = lane k's value of this lane's 8-lane group (k = 0..7): ds_swizzle
// in bit mode, lane' = (lane & 0x18) | k within each 32 lanes.
template <int K>
__device__ __forceinline__ float swz8(float v)
{
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (K << 5)));
}

__device__ __forceinline__ void group8_bcast(float v, float out[8])
{
    out[0] = swz8<0>(v); out[1] = swz8<1>(v); out[2] = swz8<2>(v); out[3] = swz8<3>(v);
    out[4] = swz8<4>(v); out[5] = swz8<5>(v); out[6] = swz8<6>(v); out[7] = swz8<7>(v);
}

// ((hi - lo) / qmax).clamp_min(1e-12): a NaN passes through, as in torch.
__device__ __forceinline__ float quant_scale(float lo, float hi, float qmax)
{
    const float s = __fdiv_rn(__fsub_rn(hi, lo), qmax);
    return s < 1e-12f ? 1e-12f : s;
}

// RN((x - lo) / s) rounded half-to-even, clamped to [0, qmax] and inserted
// as byte K of acc.
template <int K, uint32_t kBits>
__device__ __forceinline__ uint32_t quant_byte(float x, float lo, float s, float y, uint32_t acc)
{
    return insert_q<K>(div_rn(__fsub_rn(x, lo), s, y), kBits, acc);
}

__device__ __forceinline__ void unpack8(uint4 w, float x[8])
{
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        x[2 * k] = bf16_to_f32(ww[k] & 0xffffu);
        x[2 * k + 1] = bf16_to_f32(ww[k] >> 16);
    }
}

// 8 consecutive elements -> int8 bytes (2 dwords) or int4 nibbles (1 dword,
// element 2i in the low nibble).  Column-dependent parameters come in
// lo[k] / s[k] / y[k] with stride `ps` (1: per element, 0: shared).
template <int PS, uint32_t kBits>
__device__ __forceinline__ void quant8(const float x[8], const float* lo, const float* s, const float* y,
                                       uint32_t out[2])
{
    uint32_t d0 = 0, d1 = 0;
    d0 = quant_byte<0, kBits>(x[0], lo[0], s[0], y[0], d0);
    d0 = quant_byte<1, kBits>(x[1], lo[PS], s[PS], y[PS], d0);
    d0 = quant_byte<2, kBits>(x[2], lo[2 * PS], s[2 * PS], y[2 * PS], d0);
    d0 = quant_byte<3, kBits>(x[3], lo[3 * PS], s[3 * PS], y[3 * PS], d0);
    d1 = quant_byte<0, kBits>(x[4], lo[4 * PS], s[4 * PS], y[4 * PS], d1);
    d1 = quant_byte<1, kBits>(x[5], lo[5 * PS], s[5 * PS], y[5 * PS], d1);
    d1 = quant_byte<2, kBits>(x[6], lo[6 * PS], s[6 * PS], y[6 * PS], d1);
    d1 = quant_byte<3, kBits>(x[7], lo[7 * PS], s[7 * PS], y[7 * PS], d1);
    if (kBits == 8) {
        out[0] = d0;
        out[1] = d1;
    } else {
        // bytes q0..q3 (each <= 15) -> byte 0 = q0 | q1 << 4, byte 2 = q2 | q3 << 4
        const uint32_t t0 = d0 | (d0 >> 4), t1 = d1 | (d1 >> 4);
        out[0] = __builtin_amdgcn_perm(t1, t0, 0x06040200u);
        out[1] = 0;
    }
}

// Byte mask (0xff per byte to keep) of 8 consecutive int4 K elements packed
// by quant8, for a lane whose column groups are not all finite.  The
// reference packs q[2i] + 16 q[2i+1] in float before its uint8 cast
// (transport_codec.py:33-34), so a NaN quotient in either element zeroes the
// whole byte.  quant8's nibbles already equal the reference's (its
// reciprocal form may turn finite / inf into NaN where IEEE division gives
// 0, and both cast to 0); only the whole-byte rule is added here.  The IEEE
// quotient (x - lo) / s is NaN iff x - lo or s is NaN, or both are infinite
// (with finite parameters it is never NaN).
__device__ __forceinline__ uint32_t int4_nan_pairs_keep(const float x[8], const float* lo, const float* s)
{
    uint32_t keep = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        bool nan = false;
#pragma unroll
        for (int j = 2 * i; j < 2 * i + 2; ++j) {
            const float a = __fsub_rn(x[j], lo[j]);
            nan = nan || __builtin_isnan(a) || __builtin_isnan(s[j]) || (__builtin_isinf(a) && __builtin_isinf(s[j]));
        }
        keep |= (nan ? 0u : 0xffu) << (8 * i);
    }
    return keep;
}

template <uint32_t kBits>
__device__ __forceinline__ void store_q8(uint8_t* pkt, uint32_t e, const uint32_t w[2])
{
    if (kBits == 8) *reinterpret_cast<uint2*>(pkt + e) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(pkt + e / 2u) = w[0];
}

// Header {1, layer, kind, bits} closing the packet (the width is a multiple
// of 16, so there is no further padding).
__device__ __forceinline__ void store_header(const CodecBatch& b, uint8_t* pkt, uint32_t kind)
{
    *reinterpret_cast<uint4*>(pkt + b.qbytes + 2 * b.sbytes) = make_uint4(1u, b.layer, kind, b.bits);
}

// K: eight lanes per (token group of 64, 8 consecutive columns), each lane 8
// tokens held in registers; the column min / max is reduced across the eight
// lanes, so the slot is read once.  Workgroup bx of K record r.
template <uint32_t kBits>
__device__ __forceinline__ void quant_k_block(const CodecBatch& b, uint32_t r, uint32_t bx)
{
    const uint32_t hd = b.heads * b.dim;
    const uint32_t nch = hd / 8u;
    const uint32_t idx = bx * 256u + threadIdx.x;
    // Whole 8-lane groups take the same branch (shuffle partners stay active).
    if (idx >= 2u * nch * 8u) return;
    // A slot id out of range reads nothing from the cache: the record's
    // packet encodes zeros (its tag is poisoned by the encrypt kernel).
    const int64_t sid = b.slots[r];
    const bool bad = sid < 0 || sid >= b.nslots;
    const uint32_t l8 = idx & 7u, cg = idx >> 3;
    const uint32_t g = cg >= nch ? 1u : 0u;
    const uint32_t col = (cg - g * nch) * 8u;
    const float qmax = float((1u << kBits) - 1u);
    const uint8_t* slot = b.cache[0] + uint64_t(bad ? 0 : sid) * b.slot_bytes;
    uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    if (idx == 0) store_header(b, pkt, 0u);

    const uint32_t t0 = g * 64u + l8 * 8u;
    uint4 raw[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt)
        raw[tt] = bad ? make_uint4(0, 0, 0, 0)
                      : *reinterpret_cast<const uint4*>(slot + (uint64_t(t0 + tt) * hd + col) * 2u);
    float lo[8], hi[8];
    {
        float x[8];
        unpack8(raw[0], x);
#pragma unroll
        for (int k = 0; k < 8; ++k) { lo[k] = x[k]; hi[k] = x[k]; }
    }
#pragma unroll
    for (int tt = 1; tt < 8; ++tt) {
        float x[8];
        unpack8(raw[tt], x);
#pragma unroll
        for (int k = 0; k < 8; ++k) { lo[k] = nmin(lo[k], x[k]); hi[k] = nmax(hi[k], x[k]); }
    }
    // Min / max over the eight lanes of a chunk with DPP moves: swap within
    // pairs, then within quads, then mirror the 8-lane half-row.
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        lo[k] = nmin(lo[k], lane_dpp<0xb1>(lo[k]));
        hi[k] = nmax(hi[k], lane_dpp<0xb1>(hi[k]));
        lo[k] = nmin(lo[k], lane_dpp<0x4e>(lo[k]));
        hi[k] = nmax(hi[k], lane_dpp<0x4e>(hi[k]));
        lo[k] = nmin(lo[k], lane_dpp<0x141>(lo[k]));
        hi[k] = nmax(hi[k], lane_dpp<0x141>(hi[k]));
    }
    // Lane l8 forms column l8's scale and reciprocal (and stores the
    // column's parameters); the eight lanes then share them by swizzles,
    // which run on the LDS crossbar instead of the VALU.
    float lo_l = lo[0], hi_l = hi[0];
#pragma unroll
    for (int k = 1; k < 8; ++k)
        if (l8 == uint32_t(k)) { lo_l = lo[k]; hi_l = hi[k]; }
    const float sc_l = quant_scale(lo_l, hi_l, qmax);
    const float rc_l = recip_rn(sc_l);
    {
        const uint32_t p = g * hd + col + l8;
        reinterpret_cast<float*>(pkt + b.qbytes)[p] = sc_l;
        reinterpret_cast<float*>(pkt + b.qbytes + b.sbytes)[p] = lo_l;
    }
    float sc[8], rc[8];
    group8_bcast(sc_l, sc);
    group8_bcast(rc_l, rc);
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
        float x[8];
        unpack8(raw[tt], x);
        uint32_t w[2];
        quant8<1, kBits>(x, lo, sc, rc, w);
        store_q8<kBits>(pkt, (t0 + tt) * hd + col, w);
    }
    // int4 pairs two columns of different groups in one byte: a lane with a
    // non-finite group (the only way to a NaN quotient) stores its bytes
    // again under the pairwise rule (a second pass, so the common path keeps
    // its registers).
    if (kBits == 4) {
        bool finite = true;
#pragma unroll
        for (int k = 0; k < 8; ++k) finite = finite && __builtin_isfinite(lo[k]) && __builtin_isfinite(sc[k]);
        if (!finite) {
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                // read again (a rare path: keeping raw[] live would cost the
                // common path a wave per SIMD)
                uint32_t off = ((t0 + tt) * hd + col) * 2u;
                asm volatile("" : "+v"(off));  // a fresh load, not raw[tt] kept alive
                const uint4 rw = bad ? make_uint4(0, 0, 0, 0) : *reinterpret_cast<const uint4*>(slot + off);
                float x[8];
                unpack8(rw, x);
                uint32_t w[2];
                quant8<1, kBits>(x, lo, sc, rc, w);
                w[0] &= int4_nan_pairs_keep(x, lo, sc);
                store_q8<kBits>(pkt, (t0 + tt) * hd + col, w);
            }
        }
    }
}


// V: two lanes per (token, head, dim group of 64), 32 consecutive elements
// each; the group's min / max meets in one DPP swap, and the group's scale
// and reciprocal are formed once per 32 elements.  Workgroup bx of V record r.
template <uint32_t kBits>
__device__ __forceinline__ void quant_v_block(const CodecBatch& b, uint32_t r, uint32_t bx)
{
    const uint32_t hd = b.heads * b.dim;
    const uint32_t idx = bx * 256u + threadIdx.x;
    const uint32_t ngroups = 2u * hd;  // 128 * hd / 64
    // Lane pairs (2i, 2i+1) take the same branch, so the swap below always
    // meets an active partner.
    if (idx >= ngroups * 2u) return;
    const int64_t sid = b.slots[r];
    const bool bad = sid < 0 || sid >= b.nslots;  // encode zeros, as in quant_k_block
    const uint32_t gi = idx >> 1, half = idx & 1u;
    const float qmax = float((1u << kBits) - 1u);
    const uint8_t* slot = b.cache[1] + uint64_t(bad ? 0 : sid) * b.slot_bytes;
    uint8_t* pkt = b.staging + uint64_t(r) * b.staging_stride;
    if (idx == 0) store_header(b, pkt, 1u);
    const uint32_t e = gi * 64u + half * 32u;
    uint4 raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        raw[k] = bad ? make_uint4(0, 0, 0, 0) : *reinterpret_cast<const uint4*>(slot + uint64_t(e + 8u * k) * 2u);
    float x[32];
#pragma unroll
    for (int k = 0; k < 4; ++k) unpack8(raw[k], x + 8 * k);
    float lo = x[0], hi = x[0];
#pragma unroll
    for (int k = 1; k < 32; ++k) { lo = nmin(lo, x[k]); hi = nmax(hi, x[k]); }
    lo = nmin(lo, lane_dpp<0xb1>(lo));
    hi = nmax(hi, lane_dpp<0xb1>(hi));
    const float s = quant_scale(lo, hi, qmax);
    const float y = recip_rn(s);
    if (half == 0) {
        reinterpret_cast<float*>(pkt + b.qbytes)[gi] = s;
        reinterpret_cast<float*>(pkt + b.qbytes + b.sbytes)[gi] = lo;
    }
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t p2[2];
        quant8<0, kBits>(x + 8 * k, &lo, &s, &y, p2);
        w[2 * k] = p2[0];
        w[2 * k + 1] = p2[1];
    }
    if (kBits == 8) {
        uint4* dst = reinterpret_cast<uint4*>(pkt + e);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
        *reinterpret_cast<uint4*>(pkt + e / 2u) = make_uint4(w[0], w[2], w[4], w[6]);
    }
}

// Both kinds in one launch: the kx workgroups of each K record, then the vx
// of each V record.  The K blocks are bound by their strided slot reads (8
// token rows per lane), the V blocks stream; in one grid the V blocks fill
// the machine while the K blocks drain (MI355X, Llama-3-70B int4 layer: 22.7
// + 18.8 us as two launches, 6.5 us less per layer as one).
template <uint32_t kBits>
__global__ __launch_bounds__(256) void quant_kernel(CodecBatch b, uint32_t kx, uint32_t vx)
{
    clock_stamp(b.clock, 0);
    const uint32_t nkb = kx * b.n_k;
    if (blockIdx.x < nkb) {
        quant_k_block<kBits>(b, blockIdx.x / kx, blockIdx.x % kx);
    } else {
        const uint32_t v = blockIdx.x - nkb;
        quant_v_block<kBits>(b, b.n_k + v / vx, v % vx);
    }
    clock_stamp(b.clock, 1);
}

// CUs of an MI355X, the unit of the dequantiser's grid sizing.
constexpr uint64_t kCus = 256;

hipError_t launch_dequant_scatter(hipStream_t stream, const CodecBatch& b, const LaunchEvents& ev)
{
    // Tokens per thread (a power of two, 1..16): about one workgroup per CU
    // for the K records and two for the V records.  Measured on MI355X (layer
    // time with the record kernel; K, V tokens per thread): int4 Qwen2.5-7B
    // (512 columns, 64 + 64 records) 24.5 / 24.0 / 25.7 / 30.1 us at
    // (2,2) / (4,2) / (8,2) / (16,2), 25.4 at (8,4); int8 Llama-3-8B (1024
    // columns) 40.4 / 39.8 / 39.5 / 41.8 us at (2,2) / (4,2) / (8,2) /
    // (16,2), 39.5 at (8,4) -- the fastest split is 768 workgroups in both.
    // More workgroups beat sharing a K thread's (scale, low) loads over more
    // tokens.
    const uint32_t nc = b.heads * b.dim / 16u;  // 16-column chunks per token
    const auto tokens = [nc](uint32_t nrec, uint64_t wgs) {
        const uint64_t t = uint64_t(128u) * nc * nrec / (wgs * 256u);  // tokens per thread for `wgs` workgroups
        uint32_t p = 1;
        while (p < 16u && uint64_t(p) * 2u <= t) p *= 2u;
        return p;
    };
    const uint32_t tk = tokens(b.n_k, kCus), tv = tokens(b.nrec - b.n_k, 2u * kCus);
    const uint32_t kx = ((128u / tk) * nc + 255u) / 256u, vx = ((128u / tv) * nc + 255u) / 256u;
    const dim3 grid(kx * b.n_k + vx * (b.nrec - b.n_k));
    CodecBatch bb = b;
    bb.clock = ev.clock ? ev.clock->take(uint64_t(grid.x) * 4u) : nullptr;
    if (ev.start || ev.stop)
        hipExtLaunchKernelGGL(dequant_scatter_kernel, grid, dim3(256), 0, stream, ev.start, ev.stop, 0, bb, kx, vx,
                              tk, tv);
    else
        hipLaunchKernelGGL(dequant_scatter_kernel, grid, dim3(256), 0, stream, bb, kx, vx, tk, tv);
    return hipGetLastError();
}

hipError_t launch_gather_quant(hipStream_t stream, const CodecBatch& b, const LaunchEvents& ev)
{
    const uint32_t hd = b.heads * b.dim;
    const uint32_t nv = b.nrec - b.n_k;
    const uint32_t kx = (2u * hd + 255u) / 256u, vx = (4u * hd + 255u) / 256u;
    if (b.n_k + nv) {
        const dim3 grid(kx * b.n_k + vx * nv);
        CodecBatch bb = b;
        bb.clock = ev.clock ? ev.clock->take(uint64_t(grid.x) * 4u) : nullptr;
        if (ev.start || ev.stop) {
            if (bb.bits == 8)
                hipExtLaunchKernelGGL(quant_kernel<8>, grid, dim3(256), 0, stream, ev.start, ev.stop, 0, bb, kx, vx);
            else
                hipExtLaunchKernelGGL(quant_kernel<4>, grid, dim3(256), 0, stream, ev.start, ev.stop, 0, bb, kx, vx);
        } else if (bb.bits == 8) {
            hipLaunchKernelGGL(quant_kernel<8>, grid, dim3(256), 0, stream, bb, kx, vx);
        } else {
            hipLaunchKernelGGL(quant_kernel<4>, grid, dim3(256), 0, stream, bb, kx, vx);
        }
    }
    return hipGetLastError();
}

}  // namespace si
