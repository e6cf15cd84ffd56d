// Device primitives for AES-128-GCM on gfx950 (CDNA4).
//
// Data layout conventions used by every kernel:
//   * AES state and round keys are four little-endian column words, i.e. the
//     16-byte block loaded from memory as four dwords.  Column j's byte r is
//     state row r.  Te0[x] = {2s, s, s, 3s} (s = S(x)) packs MixColumns' first
//     column; Te1 = rotl8(Te0); the other two are rotl16 of these.
//   * GF(2^128) elements for GHASH are kept in memory byte order (four LE
//     dwords) wherever only XORs and table lookups touch them; the generic
//     multiply converts to big-endian words (bit 0 = MSB of byte 0 = x^0).
//
// LDS tables (per workgroup):
//   AES  : entry e, table t in {Te0, Te1}, copy c in [0, 32): 32-bit word at
//          byte address e*256 + t*128 + c*4.  Lane l reads copy (l & 31), so a
//          wave64 lookup touches each of the 32 banks once per half-wave.  The
//          address is produced by ONE v_perm_b32: byte1 <- state byte, byte0 <-
//          the lane's copy offset.
//   GHASH: 4-bit per-position tables of H^(UT), H^(2UT) (a unit's row
//          step and row pair), H^T and H^2T (combining the units' partials);
//          T = threads per unit = blocks per row, U = units per workgroup.
//          Position p (nibble p of the block, p = 0..31), value v: 16 bytes
//          at p*256 + v*16.  Y*H^e = XOR_p table[p][nibble_p(Y)].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "si_layout.h"

namespace si {

__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c)
{
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ uint32_t rotl16(uint32_t x)
{
    return __builtin_amdgcn_alignbit(x, x, 16);
}

__device__ __forceinline__ uint32_t bswap32(uint32_t x)
{
    return __builtin_amdgcn_perm(x, x, 0x00010203u);
}

// ---------------------------------------------------------------- AES

// Lane-specific byte offsets of the lane's copy of Te0 / Te1.
struct AesLane {
    uint32_t b0, b1;
};

__device__ __forceinline__ AesLane aes_lane(uint32_t lane)
{
    AesLane l;
    l.b0 = (lane & 31u) * 4u;
    l.b1 = 128u + (lane & 31u) * 4u;
    return l;
}

// Table word for byte k of state word w: one v_perm_b32 builds the address
// (byte 1 <- the state byte, byte 0 <- the lane's copy offset).
template <int K>
__device__ __forceinline__ uint32_t te(const uint32_t* lds, uint32_t w, uint32_t base)
{
    constexpr uint32_t sel = 0x0c0c0000u | ((4u + K) << 8);
    const uint32_t addr = __builtin_amdgcn_perm(w, base, sel);
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds) + addr);
}

// Te_K[byte K of w] for K = 0..3 (Te2, Te3 are rotl16 of Te0, Te1).
template <int K>
__device__ __forceinline__ uint32_t te_full(const uint32_t* lds, uint32_t w, AesLane l)
{
    const uint32_t v = te<K>(lds, w, (K & 1) ? l.b1 : l.b0);
    return K >= 2 ? rotl16(v) : v;
}

// Fills the AES region (64 KiB) from Te0 with 256 threads: thread e writes
// the 16 columns of entry e (columns 0..7 hold Te0 copies, 8..15 Te1 copies),
// starting at column e & 15 so a wave's stores spread over all banks.
__device__ __forceinline__ void aes_fill_lds(uint32_t* lds, const uint32_t* __restrict__ te0,
                                             uint32_t tid)
{
    static_assert(SI_T == 256, "one Te0 entry per thread");
    const uint32_t v0 = te0[tid];
    const uint32_t v1 = __builtin_amdgcn_alignbit(v0, v0, 24);  // rotl8
    uint4* dst = reinterpret_cast<uint4*>(lds) + tid * 16u;
#pragma unroll
    for (uint32_t c = 0; c < 16; ++c) {
        const uint32_t col = (c + tid) & 15u;
        const uint32_t v = (col & 8u) ? v1 : v0;
        dst[col] = make_uint4(v, v, v, v);
    }
}

// Round keys held in VGPRs for the whole kernel: rk16 of rounds 1..9 and the
// plain last-round key.  Loaded through an opaque per-lane zero so the compiler
// keeps them in vector registers instead of reloading scalars in the loop.
struct AesKeys {
    uint32_t rk3;
    uint32_t r16[36];   // rk16[4..39]
    uint32_t last[4];   // rk[40..43]
};

__device__ __forceinline__ void load_keys(const GcmCtx* __restrict__ ctx, AesKeys& k)
{
    uint32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    const uint4* p16 = reinterpret_cast<const uint4*>(ctx->rk16 + 4) + z;
#pragma unroll
    for (int i = 0; i < 9; ++i) {
        const uint4 q = p16[i];
        k.r16[4 * i] = q.x; k.r16[4 * i + 1] = q.y; k.r16[4 * i + 2] = q.z; k.r16[4 * i + 3] = q.w;
    }
    const uint4 q = reinterpret_cast<const uint4*>(ctx->rk + 40)[z];
    k.last[0] = q.x; k.last[1] = q.y; k.last[2] = q.z; k.last[3] = q.w;
    k.rk3 = ctx->rk[3 + z];
}

// Rounds `r0`..9 and the last round from state s.
__device__ __forceinline__ void aes_rounds(const uint32_t* lds, AesLane l, const AesKeys& k,
                                           int r0, uint32_t s0, uint32_t s1, uint32_t s2,
                                           uint32_t s3, uint32_t out[4])
{
#pragma unroll
    for (int r = 1; r <= 9; ++r) {
        if (r < r0) continue;
        const uint32_t* rk = k.r16 + 4 * (r - 1);
        const uint32_t t0 = xor3(te<0>(lds, s0, l.b0), te<1>(lds, s1, l.b1),
                                 rotl16(xor3(te<2>(lds, s2, l.b0), te<3>(lds, s3, l.b1), rk[0])));
        const uint32_t t1 = xor3(te<0>(lds, s1, l.b0), te<1>(lds, s2, l.b1),
                                 rotl16(xor3(te<2>(lds, s3, l.b0), te<3>(lds, s0, l.b1), rk[1])));
        const uint32_t t2 = xor3(te<0>(lds, s2, l.b0), te<1>(lds, s3, l.b1),
                                 rotl16(xor3(te<2>(lds, s0, l.b0), te<3>(lds, s1, l.b1), rk[2])));
        const uint32_t t3 = xor3(te<0>(lds, s3, l.b0), te<1>(lds, s0, l.b1),
                                 rotl16(xor3(te<2>(lds, s1, l.b0), te<3>(lds, s2, l.b1), rk[3])));
        s0 = t0; s1 = t1; s2 = t2; s3 = t3;
    }
    // Last round: S-box bytes sit in byte 1 of Te0 and byte 2 of Te1.
    // (lo | hi) ^ rk : bitop3 truth table 0x56.
#define SI_LAST(J, A, B, C, D)                                                            \
    out[J] = __builtin_amdgcn_bitop3_b32(                                                  \
        __builtin_amdgcn_perm(te<0>(lds, A, l.b0), te<1>(lds, B, l.b1), 0x0c0c0205u),     \
        __builtin_amdgcn_perm(te<2>(lds, C, l.b0), te<3>(lds, D, l.b1), 0x02050c0cu),     \
        k.last[J], 0x56)
    SI_LAST(0, s0, s1, s2, s3);
    SI_LAST(1, s1, s2, s3, s0);
    SI_LAST(2, s2, s3, s0, s1);
    SI_LAST(3, s3, s0, s1, s2);
#undef SI_LAST
}

// E_K(counter block) with the three nonce words already XORed with rk[0..2].
__device__ __forceinline__ void aes_ctr_block(const uint32_t* lds, AesLane l, const AesKeys& k,
                                              uint32_t n0, uint32_t n1, uint32_t n2, uint32_t ctr,
                                              uint32_t out[4])
{
    aes_rounds(lds, l, k, 1, n0, n1, n2, bswap32(ctr) ^ k.rk3, out);
}

// Counter-mode cache of rounds 1 and 2 (valid while counter bytes 12..13 stay
// fixed and byte 15 is the same for all of a thread's blocks, i.e. its blocks
// are 256*q apart).  With state word 3 = bswap(ctr) ^ rk3 the only byte that
// moves between the thread's blocks is s3.b2 (counter byte 14); round 1 then
// reduces to one lookup and round 2 to four:
//   t1 = U1 ^ Te2[s3.b2],  v = C ^ {Te1[t1.b1], Te0[t1.b0], Te3[t1.b3], Te2[t1.b2]}.
struct CtrCache {
    uint32_t u1, c0, c1, c2, c3;
};

__device__ __forceinline__ CtrCache ctr_cache(const uint32_t* lds, AesLane l,
                                              const GcmCtx* __restrict__ ctx, uint32_t n0,
                                              uint32_t n1, uint32_t n2, uint32_t s3)
{
    const uint32_t* rk = ctx->rk;
    const uint32_t u0 = te_full<0>(lds, n0, l) ^ te_full<1>(lds, n1, l) ^ te_full<2>(lds, n2, l) ^
                        te_full<3>(lds, s3, l) ^ rk[4];
    const uint32_t u2 = te_full<0>(lds, n2, l) ^ te_full<1>(lds, s3, l) ^ te_full<2>(lds, n0, l) ^
                        te_full<3>(lds, n1, l) ^ rk[6];
    const uint32_t u3 = te_full<0>(lds, s3, l) ^ te_full<1>(lds, n0, l) ^ te_full<2>(lds, n1, l) ^
                        te_full<3>(lds, n2, l) ^ rk[7];
    CtrCache c;
    c.u1 = te_full<0>(lds, n1, l) ^ te_full<1>(lds, n2, l) ^ te_full<3>(lds, n0, l) ^ rk[5];
    c.c0 = te_full<0>(lds, u0, l) ^ te_full<2>(lds, u2, l) ^ te_full<3>(lds, u3, l) ^ rk[8];
    c.c1 = te_full<1>(lds, u2, l) ^ te_full<2>(lds, u3, l) ^ te_full<3>(lds, u0, l) ^ rk[9];
    c.c2 = te_full<0>(lds, u2, l) ^ te_full<1>(lds, u3, l) ^ te_full<2>(lds, u0, l) ^ rk[10];
    c.c3 = te_full<0>(lds, u3, l) ^ te_full<1>(lds, u0, l) ^ te_full<3>(lds, u2, l) ^ rk[11];
    return c;
}

__device__ __forceinline__ void aes_ctr_block_cached(const uint32_t* lds, AesLane l,
                                                     const AesKeys& k, const CtrCache& c,
                                                     uint32_t ctr, uint32_t out[4])
{
    const uint32_t s3 = bswap32(ctr) ^ k.rk3;
    const uint32_t t1 = c.u1 ^ rotl16(te<2>(lds, s3, l.b0));
    const uint32_t v0 = c.c0 ^ te<1>(lds, t1, l.b1);
    const uint32_t v1 = c.c1 ^ te<0>(lds, t1, l.b0);
    const uint32_t v2 = c.c2 ^ rotl16(te<3>(lds, t1, l.b1));
    const uint32_t v3 = c.c3 ^ rotl16(te<2>(lds, t1, l.b0));
    aes_rounds(lds, l, k, 3, v0, v1, v2, v3, out);
}

// ---------------------------------------------------------------- GHASH

// Table reads of one AES round of state s: q[4j + K] = Te_K-source for
// column j (byte K of word j+K), not yet rotated.
__device__ __forceinline__ void aes_issue(const uint32_t* lds, AesLane l, const uint32_t s[4],
                                          uint32_t q[16])
{
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        q[4 * j + 0] = te<0>(lds, s[j], l.b0);
        q[4 * j + 1] = te<1>(lds, s[(j + 1) & 3], l.b1);
        q[4 * j + 2] = te<2>(lds, s[(j + 2) & 3], l.b0);
        q[4 * j + 3] = te<3>(lds, s[(j + 3) & 3], l.b1);
    }
}

// Round output from the reads of aes_issue and the pre-rotated round key.
__device__ __forceinline__ void aes_combine(const uint32_t q[16], const uint32_t* rk16, uint32_t s[4])
{
#pragma unroll
    for (int j = 0; j < 4; ++j)
        s[j] = xor3(q[4 * j], q[4 * j + 1], rotl16(xor3(q[4 * j + 2], q[4 * j + 3], rk16[j])));
}

// Last round from the reads of aes_issue: S-box bytes sit in byte 1 of Te0 and
// byte 2 of Te1; (lo | hi) ^ rk is bitop3 truth table 0x56.
__device__ __forceinline__ void aes_combine_last(const uint32_t q[16], const uint32_t* rk,
                                                 uint32_t out[4])
{
#pragma unroll
    for (int j = 0; j < 4; ++j)
        out[j] = __builtin_amdgcn_bitop3_b32(__builtin_amdgcn_perm(q[4 * j], q[4 * j + 1], 0x0c0c0205u),
                                             __builtin_amdgcn_perm(q[4 * j + 2], q[4 * j + 3], 0x02050c0cu),
                                             rk[j], 0x56);
}

// Byte offset (nibble * 16) of 4-bit position P of the 128-bit value `in`
// in P's 256-byte table: position P = 8w + 2b + h is the low (h = 0) or high
// (h = 1) nibble of byte b of word w.  One SDWA instruction each:
//   low:  (byte_b << 4) truncated to a byte = low nibble * 16;
//   high: byte_b & 0xf0 = high nibble * 16.
template <int P>
__device__ __forceinline__ uint32_t nib_off(const uint32_t in[4])
{
    constexpr int w = P >> 3, b = (P & 7) >> 1;
    const uint32_t x = in[w];
    uint32_t d;
#define SI_NIB_LO(B)                                                                              \
    asm volatile("v_lshlrev_b32_sdwa %0, 4, %1 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD "        \
        "src1_sel:BYTE_" #B : "=v"(d) : "v"(x))
#define SI_NIB_HI(B)                                                                              \
    asm volatile("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_" #B          \
        " src1_sel:DWORD" : "=v"(d) : "v"(x), "s"(0xf0u))
    if constexpr (P & 1) {
        if constexpr (b == 0) SI_NIB_HI(0);
        else if constexpr (b == 1) SI_NIB_HI(1);
        else if constexpr (b == 2) SI_NIB_HI(2);
        else SI_NIB_HI(3);
    } else {
        if constexpr (b == 0) SI_NIB_LO(0);
        else if constexpr (b == 1) SI_NIB_LO(1);
        else if constexpr (b == 2) SI_NIB_LO(2);
        else SI_NIB_LO(3);
    }
#undef SI_NIB_LO
#undef SI_NIB_HI
    return d;
}

template <int P>
__device__ __forceinline__ uint4 gh_read(const char* base, const uint32_t in[4])
{
    return *reinterpret_cast<const uint4*>(base + P * 256 + nib_off<P>(in));
}

template <int P, int P1>
__device__ __forceinline__ void gh_issue_at(const char* base, const uint32_t in[4], uint4 g[])
{
    if constexpr (P < P1) {
        g[0] = gh_read<P>(base, in);
        gh_issue_at<P + 1, P1>(base, in, g + 1);
    }
}

// Reads [P0, P1) of in * H^k (4-bit per-position tables) into g.
template <int P0, int P1>
__device__ __forceinline__ void gh_issue(const uint4* tbl, const uint32_t in[4], uint4 g[])
{
    gh_issue_at<P0, P1>(reinterpret_cast<const char*>(tbl), in, g);
}

template <int N>
__device__ __forceinline__ void gh_fold(const uint4 g[], uint32_t acc[4])
{
    static_assert(N % 2 == 0, "pairs");
#pragma unroll
    for (int i = 0; i < N; i += 2) {
        acc[0] = xor3(acc[0], g[i].x, g[i + 1].x);
        acc[1] = xor3(acc[1], g[i].y, g[i + 1].y);
        acc[2] = xor3(acc[2], g[i].z, g[i + 1].z);
        acc[3] = xor3(acc[3], g[i].w, g[i + 1].w);
    }
}

#define SI_STAGE() __builtin_amdgcn_sched_barrier(0)

// Keystreams of two counter blocks (counter-mode cache of rounds 1-2) and the
// GHASH fold of a ciphertext row pair, acc = y*H^2T ^ xa*H^T, software
// pipelined by hand: each stage consumes reads issued two stages earlier and
// issues the next ones, and scheduling barriers keep the stages apart, so a
// wave keeps its LDS queue (15 reads) full instead of draining it every few
// reads.  Stage order per AES round r: GHASH slice, combine A(r-1) + issue
// A(r), combine B(r-1) + issue B(r).
__device__ __forceinline__ void ctr2_ghash2(const uint32_t* lds, AesLane l, const AesKeys& k,
                                            const CtrCache& c, uint32_t ctr_a, uint32_t ctr_b,
                                            const uint4* gh, const uint4* gh2, const uint32_t y[4],
                                            const uint32_t xa[4], uint32_t ks_a[4],
                                            uint32_t ks_b[4], uint32_t acc[4])
{
    acc[0] = acc[1] = acc[2] = acc[3] = 0;
    uint32_t a[4], b[4], qa[16], qb[16];
    uint4 g0[8], g1[8];
    uint32_t ra, rb, ta, tb;
    // Round 1: one varying read per block.
    ra = te<2>(lds, bswap32(ctr_a) ^ k.rk3, l.b0);
    rb = te<2>(lds, bswap32(ctr_b) ^ k.rk3, l.b0);
    gh_issue<0, 8>(gh2, y, g0);
    SI_STAGE();
    // Round 2: four varying reads per block.
    ta = c.u1 ^ rotl16(ra);
    qa[0] = te<1>(lds, ta, l.b1); qa[1] = te<0>(lds, ta, l.b0);
    qa[2] = te<3>(lds, ta, l.b1); qa[3] = te<2>(lds, ta, l.b0);
    tb = c.u1 ^ rotl16(rb);
    qb[0] = te<1>(lds, tb, l.b1); qb[1] = te<0>(lds, tb, l.b0);
    qb[2] = te<3>(lds, tb, l.b1); qb[3] = te<2>(lds, tb, l.b0);
    SI_STAGE();
    gh_fold<8>(g0, acc);
    gh_issue<8, 16>(gh2, y, g1);
    SI_STAGE();
    a[0] = c.c0 ^ qa[0]; a[1] = c.c1 ^ qa[1]; a[2] = c.c2 ^ rotl16(qa[2]); a[3] = c.c3 ^ rotl16(qa[3]);
    aes_issue(lds, l, a, qa);
    SI_STAGE();
    b[0] = c.c0 ^ qb[0]; b[1] = c.c1 ^ qb[1]; b[2] = c.c2 ^ rotl16(qb[2]); b[3] = c.c3 ^ rotl16(qb[3]);
    aes_issue(lds, l, b, qb);
    SI_STAGE();
#define SI_ROUND(R, FOLD_N, FOLD_G, ISSUE)                                \
    gh_fold<FOLD_N>(FOLD_G, acc);                                         \
    ISSUE;                                                                \
    SI_STAGE();                                                           \
    aes_combine(qa, k.r16 + 4 * ((R) - 1), a);                            \
    aes_issue(lds, l, a, qa);                                             \
    SI_STAGE();                                                           \
    aes_combine(qb, k.r16 + 4 * ((R) - 1), b);                            \
    aes_issue(lds, l, b, qb);                                             \
    SI_STAGE();
    SI_ROUND(3, 8, g1, (gh_issue<16, 22>(gh2, y, g0)))
    SI_ROUND(4, 6, g0, (gh_issue<22, 30>(gh2, y, g1)))
    SI_ROUND(5, 8, g1, (gh_issue<30, 32>(gh2, y, g0), gh_issue<0, 6>(gh, xa, g0 + 2)))
    SI_ROUND(6, 8, g0, (gh_issue<6, 12>(gh, xa, g1)))
    SI_ROUND(7, 6, g1, (gh_issue<12, 20>(gh, xa, g0)))
    SI_ROUND(8, 8, g0, (gh_issue<20, 26>(gh, xa, g1)))
    SI_ROUND(9, 6, g1, (gh_issue<26, 32>(gh, xa, g0)))
#undef SI_ROUND
    aes_combine_last(qa, k.last, ks_a);
    aes_combine_last(qb, k.last, ks_b);
    gh_fold<6>(g0, acc);
}

// out = in * H^k with the 4-bit per-position tables of H^k in LDS (position
// p's 256-byte table is the instruction's immediate offset).  For word w of
// `in`, L = (w << 4) & 0xf0f0f0f0 and H = w & 0xf0f0f0f0 hold nibble*16 of
// every low / high nibble in their own bytes, so each lookup address is one
// byte extract.
__device__ __forceinline__ void gh_mul(const uint4* tbl, const uint32_t in[4], uint32_t out[4])
{
    uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
    const char* base = reinterpret_cast<const char*>(tbl);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t lo = (in[w] << 4) & 0xf0f0f0f0u;
        const uint32_t hi = in[w] & 0xf0f0f0f0u;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int p = 8 * w + 2 * b;
            const uint32_t ol = (lo >> (8 * b)) & 0xffu;
            const uint32_t oh = (hi >> (8 * b)) & 0xffu;
            const uint4 v0 = *reinterpret_cast<const uint4*>(base + p * 256 + ol);
            const uint4 v1 = *reinterpret_cast<const uint4*>(base + (p + 1) * 256 + oh);
            a0 = xor3(a0, v0.x, v1.x);
            a1 = xor3(a1, v0.y, v1.y);
            a2 = xor3(a2, v0.z, v1.z);
            a3 = xor3(a3, v0.w, v1.w);
        }
    }
    out[0] = a0; out[1] = a1; out[2] = a2; out[3] = a3;
}

// y <- y * H^k
__device__ __forceinline__ void gh_mul_table(const uint4* tbl, uint32_t y[4])
{
    uint32_t t[4];
    gh_mul(tbl, y, t);
    y[0] = t[0]; y[1] = t[1]; y[2] = t[2]; y[3] = t[3];
}

// Big-endian-word GF(2^128) helpers (bit 0 = MSB of word 0 = x^0).
__device__ __forceinline__ void be_mulx(uint32_t a[4])
{
    const uint32_t carry = a[3] & 1u;
    a[3] = __builtin_amdgcn_alignbit(a[2], a[3], 1);
    a[2] = __builtin_amdgcn_alignbit(a[1], a[2], 1);
    a[1] = __builtin_amdgcn_alignbit(a[0], a[1], 1);
    a[0] = (a[0] >> 1) ^ ((0u - carry) & 0xe1000000u);
}

// z = x * y for per-lane x, y (memory byte order in and out), shared by K
// threads (K = 2 or 3): Shoup's 4-bit method with a per-lane table of the
// multiples v*y in LDS.  Each thread writes its share of the table (entries
// v = c, c+K, ... for c = 0..K-1; v = 0 is not stored: entry v >= 1 sits at
// tbl[(v - 1) * stride + slot] and a shared zero word stands for v = 0), and
// after a barrier each evaluates the nibbles j = c (mod K) of x with its own
// Horner chain (step x^(4K)), then shifts by x^(4c).  XORing the K results
// gives x * y; each chain is 1/K as long as one whole product's.
template <int K>
__device__ __forceinline__ void gh_table_share(const uint32_t y_mem[4], uint32_t c, uint4* tbl,
                                               uint32_t slot, uint32_t stride)
{
    uint32_t m8[4] = {bswap32(y_mem[0]), bswap32(y_mem[1]), bswap32(y_mem[2]), bswap32(y_mem[3])};
    uint32_t m4[4] = {m8[0], m8[1], m8[2], m8[3]};
    be_mulx(m4);
    uint32_t m2[4] = {m4[0], m4[1], m4[2], m4[3]};
    be_mulx(m2);
    uint32_t m1[4] = {m2[0], m2[1], m2[2], m2[3]};
    be_mulx(m1);
#pragma unroll
    for (uint32_t i = 0; i < (16u + K - 1u) / K; ++i) {
        const uint32_t v = c + uint32_t(K) * i;
        if (v != 0u && v < 16u) {
            const uint32_t s8 = 0u - ((v >> 3) & 1u), s4 = 0u - ((v >> 2) & 1u);
            const uint32_t s2 = 0u - ((v >> 1) & 1u), s1 = 0u - (v & 1u);
            uint32_t e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) e[k] = (m8[k] & s8) ^ (m4[k] & s4) ^ (m2[k] & s2) ^ (m1[k] & s1);
            tbl[(v - 1u) * stride + slot] = make_uint4(e[0], e[1], e[2], e[3]);
        }
    }
}

// a <- a * x^S (big-endian words, S = 4 or 12): shift right by S and fold the
// S bits that left x^127 back in, x^(128+i) = x^i (x^7 + x^2 + x + 1).
template <int S>
__device__ __forceinline__ void be_mulx_s(uint32_t a[4])
{
    static_assert(S == 4 || S == 8 || S == 12, "reduction fits the top word");
    const uint32_t rem = a[3] & ((1u << S) - 1u);
    a[3] = __builtin_amdgcn_alignbit(a[2], a[3], S);
    a[2] = __builtin_amdgcn_alignbit(a[1], a[2], S);
    a[1] = __builtin_amdgcn_alignbit(a[0], a[1], S);
    const uint32_t red = (rem << (25 - S)) ^ xor3(rem << (30 - S), rem << (31 - S), rem << (32 - S));
    a[0] = (a[0] >> S) ^ red;
}

// Part C of x * y (C < K) for NS independent products at once (their
// chains interleave): z[s] = XOR_{j = C mod K} T_s[nibble j of x[s]] * x^(4j),
// Horner over those nibbles with step x^(4K).  K = 1 is the whole product,
// K = 2 or 3 a half or a third of it (gh_table_share's layout: entry v >= 1 at
// tbl[(v - 1) * stride + slot], `zero` for v = 0).
template <int K, int C, int NS>
__device__ __forceinline__ void gh_mul_part(const uint32_t (&x_mem)[NS][4], const uint4* const (&tbl)[NS],
                                            const uint4* zero, uint32_t slot, uint32_t stride,
                                            uint32_t (&z_mem)[NS][4])
{
    static_assert((K == 1 || K == 2 || K == 3) && C < K, "one, two or three parts");
    constexpr int kTop = C + K * ((31 - C) / K);
    uint32_t xb[NS][4], a[NS][4];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int k = 0; k < 4; ++k) xb[s][k] = bswap32(x_mem[s][k]);
    const auto entry = [&](int s, int j) -> const uint4* {
        const uint32_t v = (xb[s][j >> 3] >> (28 - 4 * (j & 7))) & 0xfu;
        return v ? tbl[s] + ((v - 1u) * stride + slot) : zero;
    };
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const uint4 q = *entry(s, kTop);
        a[s][0] = q.x; a[s][1] = q.y; a[s][2] = q.z; a[s][3] = q.w;
    }
#pragma unroll
    for (int j = kTop - K; j >= C; j -= K) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint4 q = *entry(s, j);
            be_mulx_s<4 * K>(a[s]);
            a[s][0] ^= q.x; a[s][1] ^= q.y; a[s][2] ^= q.z; a[s][3] ^= q.w;
        }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int i = 0; i < C; ++i) be_mulx_s<4>(a[s]);
#pragma unroll
        for (int k = 0; k < 4; ++k) z_mem[s][k] = bswap32(a[s][k]);
    }
}

// GF(2^128) product of two elements in memory byte order held as four
// little-endian words (SP 800-38D Algorithm 1), bit-serial: for the rare
// general products (set-up work, the GHASH mirror), not for the rows.
__device__ inline uint4 gf_mul4(uint4 x, uint4 y)
{
    const uint32_t xw[4] = {x.x, x.y, x.z, x.w}, yw[4] = {y.x, y.y, y.z, y.w};
    uint64_t vh = 0, vl = 0, zh = 0, zl = 0;
    for (int i = 0; i < 8; ++i) {
        vh = vh << 8 | ((yw[i >> 2] >> (8 * (i & 3))) & 0xff);
        vl = vl << 8 | ((yw[2 + (i >> 2)] >> (8 * (i & 3))) & 0xff);
    }
    for (int i = 0; i < 128; ++i) {
        const uint32_t byte = (xw[i >> 5] >> (8 * ((i >> 3) & 3))) & 0xff;
        if ((byte >> (7 - (i & 7))) & 1) {
            zh ^= vh;
            zl ^= vl;
        }
        const uint64_t lsb = vl & 1;
        vl = (vl >> 1) | (vh << 63);
        vh >>= 1;
        if (lsb) vh ^= 0xe100000000000000ull;
    }
    uint32_t z[4] = {0, 0, 0, 0};
    for (int i = 0; i < 8; ++i) {
        z[i >> 2] |= uint32_t((zh >> (56 - 8 * i)) & 0xff) << (8 * (i & 3));
        z[2 + (i >> 2)] |= uint32_t((zl >> (56 - 8 * i)) & 0xff) << (8 * (i & 3));
    }
    return make_uint4(z[0], z[1], z[2], z[3]);
}

// XOR of four words over a wave64, valid in lane 63, by DPP moves only (no
// LDS crossbar round trips): swap within pairs and quads, mirror 8 and 16
// lanes (every lane then holds its row's XOR), then row_bcast:15 into rows 1
// and 3 and row_bcast:31 into rows 2 and 3.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_xor(uint32_t v)
{
    return v ^ uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kCtrl, kRowMask, 0xf, false));
}

__device__ __forceinline__ void wave_xor4_to63(uint32_t v[4])
{
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t x = v[k];
        x = dpp_xor<0xb1, 0xf>(x);   // quad_perm [1,0,3,2]
        x = dpp_xor<0x4e, 0xf>(x);   // quad_perm [2,3,0,1]
        x = dpp_xor<0x141, 0xf>(x);  // row_half_mirror
        x = dpp_xor<0x140, 0xf>(x);  // row_mirror
        x = dpp_xor<0x142, 0xa>(x);  // row_bcast:15 -> rows 1, 3
        x = dpp_xor<0x143, 0xc>(x);  // row_bcast:31 -> rows 2, 3
        v[k] = x;
    }
}

}  // namespace si
