// Session key agreement and context set-up on the device (gfx950).
//
// The reference's device session (secure_infer.cpp:447-521 with the device
// half in kernels/aicpu/key_agreement.aicpu:9-49) derives the AES-128 key on
// the accelerator from an X25519 exchange, so the key never crosses PCIe.
// The AICPU there is a general-purpose core; here the device half is one
// wavefront of a HIP kernel:
//
//  * device entropy: the 32-byte X25519 secret is BLAKE2b over a pool of
//    clock samples taken by racing waves on every CU (the cycles each lane
//    spends on contended atomics) and over a host seed.  HIP exposes no
//    device random source; the pool never leaves device memory, so a PCIe
//    observer sees the seed but not the secret.  This is timing jitter, not
//    a certified entropy source.
//  * agree_kernel: device public = X25519(secret, 9), shared =
//    X25519(secret, host public), key = BLAKE2b-16 keyed by shared over
//    info || host public || device public || challenge, proof = BLAKE2b-32
//    keyed by key over the challenge (key_agreement.aicpu:29-44).  Only the
//    public value, the proof and a status word are copied back.
//  * ctx_build_kernel: the record kernels' context (round keys, H, the powers
//    of H and the 4-bit GHASH tables of H^T, H^2T, H^UT, H^2UT) built from
//    the device-resident key, in the layout the host builder writes.
//
// X25519 follows RFC 7748 section 5 (Montgomery ladder over GF(2^255 - 19),
// radix-2^16 limbs in 64-bit integers); BLAKE2b follows RFC 7693 (keyed, 12
// rounds).  Neither is performance-relevant: they run once per session.
#include "si_kernels.h"
#include "si_device.h"

#include <hip/hip_runtime.h>

namespace si {
namespace {

// ---------------------------------------------------------------- BLAKE2b

struct B2b {
    uint64_t h[8];
    uint64_t t;          // bytes compressed so far (messages here stay below 2^64)
    uint8_t buf[128];
    uint32_t fill;
    uint32_t out_len;
};

__device__ const uint64_t kB2bIv[8] = {0x6a09e667f3bcc908ull, 0xbb67ae8584caa73bull, 0x3c6ef372fe94f82bull,
                                       0xa54ff53a5f1d36f1ull, 0x510e527fade682d1ull, 0x9b05688c2b3e6c1full,
                                       0x1f83d9abfb41bd6bull, 0x5be0cd19137e2179ull};

__device__ const uint8_t kB2bSigma[12][16] = {
    {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15}, {14, 10, 4, 8, 9, 15, 13, 6, 1, 12, 0, 2, 11, 7, 5, 3},
    {11, 8, 12, 0, 5, 2, 15, 13, 10, 14, 3, 6, 7, 1, 9, 4}, {7, 9, 3, 1, 13, 12, 11, 14, 2, 6, 5, 10, 4, 0, 15, 8},
    {9, 0, 5, 7, 2, 4, 10, 15, 14, 1, 11, 12, 6, 8, 3, 13}, {2, 12, 6, 10, 0, 11, 8, 3, 4, 13, 7, 5, 15, 14, 1, 9},
    {12, 5, 1, 15, 14, 13, 4, 10, 0, 7, 6, 3, 9, 2, 8, 11}, {13, 11, 7, 14, 12, 1, 3, 9, 5, 0, 15, 4, 8, 6, 2, 10},
    {6, 15, 14, 9, 11, 3, 0, 8, 12, 2, 13, 7, 1, 4, 10, 5}, {10, 2, 8, 4, 7, 6, 1, 5, 15, 11, 9, 14, 3, 12, 13, 0},
    {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15}, {14, 10, 4, 8, 9, 15, 13, 6, 1, 12, 0, 2, 11, 7, 5, 3}};

__device__ __forceinline__ uint64_t rotr64(uint64_t x, int n) { return (x >> n) | (x << (64 - n)); }

__device__ void b2b_compress(B2b& s, bool last)
{
    uint64_t m[16], v[16];
    for (int i = 0; i < 16; ++i) {
        uint64_t w = 0;
        for (int b = 7; b >= 0; --b) w = (w << 8) | s.buf[8 * i + b];
        m[i] = w;
    }
    for (int i = 0; i < 8; ++i) {
        v[i] = s.h[i];
        v[i + 8] = kB2bIv[i];
    }
    v[12] ^= s.t;
    if (last) v[14] = ~v[14];
    for (int r = 0; r < 12; ++r) {
        const uint8_t* sg = kB2bSigma[r];
        // the eight mixings of a round: columns, then diagonals
        const int idx[8][4] = {{0, 4, 8, 12}, {1, 5, 9, 13}, {2, 6, 10, 14}, {3, 7, 11, 15},
                               {0, 5, 10, 15}, {1, 6, 11, 12}, {2, 7, 8, 13}, {3, 4, 9, 14}};
        for (int g = 0; g < 8; ++g) {
            uint64_t& a = v[idx[g][0]];
            uint64_t& b = v[idx[g][1]];
            uint64_t& c = v[idx[g][2]];
            uint64_t& d = v[idx[g][3]];
            a = a + b + m[sg[2 * g]];
            d = rotr64(d ^ a, 32);
            c = c + d;
            b = rotr64(b ^ c, 24);
            a = a + b + m[sg[2 * g + 1]];
            d = rotr64(d ^ a, 16);
            c = c + d;
            b = rotr64(b ^ c, 63);
        }
    }
    for (int i = 0; i < 8; ++i) s.h[i] ^= v[i] ^ v[i + 8];
}

__device__ void b2b_update(B2b& s, const uint8_t* p, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) {
        if (s.fill == 128) {  // a full block is compressed only once more input follows
            s.t += 128;
            b2b_compress(s, false);
            s.fill = 0;
        }
        s.buf[s.fill++] = p[i];
    }
}

__device__ void b2b_init(B2b& s, const uint8_t* key, uint32_t key_len, uint32_t out_len)
{
    for (int i = 0; i < 8; ++i) s.h[i] = kB2bIv[i];
    s.h[0] ^= 0x01010000ull ^ (uint64_t(key_len) << 8) ^ out_len;
    s.t = 0;
    s.fill = 0;
    s.out_len = out_len;
    if (key_len) {
        uint8_t block[128];
        for (int i = 0; i < 128; ++i) block[i] = i < int(key_len) ? key[i] : 0;
        b2b_update(s, block, 128);
    }
}

__device__ void b2b_final(B2b& s, uint8_t* out)
{
    s.t += s.fill;
    for (uint32_t i = s.fill; i < 128; ++i) s.buf[i] = 0;
    b2b_compress(s, true);
    for (uint32_t i = 0; i < s.out_len; ++i) out[i] = uint8_t(s.h[i >> 3] >> (8 * (i & 7)));
}

// ---------------------------------------------------------------- X25519

// Elements of GF(2^255 - 19) as 16 signed radix-2^16 limbs (value = sum
// l[i] * 2^(16 i)); 2^256 = 38 (mod p) folds the top half of a product.
struct Fe {
    int64_t l[16];
};

__device__ void fe_carry(Fe& a)
{
    for (int i = 0; i < 16; ++i) {
        const int64_t c = a.l[i] >> 16;  // floor division (arithmetic shift)
        a.l[i] -= c * 65536;
        if (i < 15)
            a.l[i + 1] += c;
        else
            a.l[0] += 38 * c;
    }
}

__device__ void fe_add(Fe& o, const Fe& a, const Fe& b)
{
    for (int i = 0; i < 16; ++i) o.l[i] = a.l[i] + b.l[i];
}

__device__ void fe_sub(Fe& o, const Fe& a, const Fe& b)
{
    for (int i = 0; i < 16; ++i) o.l[i] = a.l[i] - b.l[i];
}

__device__ void fe_mul(Fe& o, const Fe& a, const Fe& b)
{
    int64_t t[31];
    for (int i = 0; i < 31; ++i) t[i] = 0;
    for (int i = 0; i < 16; ++i)
        for (int j = 0; j < 16; ++j) t[i + j] += a.l[i] * b.l[j];
    for (int i = 0; i < 15; ++i) t[i] += 38 * t[i + 16];
    for (int i = 0; i < 16; ++i) o.l[i] = t[i];
    fe_carry(o);
    fe_carry(o);
}

__device__ void fe_mul_small(Fe& o, const Fe& a, int64_t k)
{
    for (int i = 0; i < 16; ++i) o.l[i] = a.l[i] * k;
    fe_carry(o);
    fe_carry(o);
}

// Constant-time swap of (a, b) when bit == 1.
__device__ void fe_cswap(Fe& a, Fe& b, int64_t bit)
{
    const int64_t mask = -bit;
    for (int i = 0; i < 16; ++i) {
        const int64_t x = mask & (a.l[i] ^ b.l[i]);
        a.l[i] ^= x;
        b.l[i] ^= x;
    }
}

// a^(p - 2): p - 2 = 2^255 - 21 has every bit set from 254 down to 0 except
// bits 4 and 2.
__device__ void fe_invert(Fe& o, const Fe& a)
{
    Fe c = a;
    for (int bit = 253; bit >= 0; --bit) {
        fe_mul(c, c, c);
        if (bit != 4 && bit != 2) fe_mul(c, c, a);
    }
    o = c;
}

__device__ void fe_unpack(Fe& o, const uint8_t in[32])
{
    for (int i = 0; i < 16; ++i) o.l[i] = int64_t(in[2 * i]) | (int64_t(in[2 * i + 1]) << 8);
    o.l[15] &= 0x7fff;  // the top bit of u is ignored (RFC 7748 section 5)
}

// Fully reduced little-endian bytes.
__device__ void fe_pack(uint8_t out[32], const Fe& a)
{
    Fe t = a;
    fe_carry(t);
    fe_carry(t);
    fe_carry(t);
    // t < 2^256 + small with limbs in [0, 2^16): subtract p while t >= p
    for (int pass = 0; pass < 2; ++pass) {
        Fe m;
        m.l[0] = t.l[0] - 0xffed;
        for (int i = 1; i < 15; ++i) {
            m.l[i] = t.l[i] - 0xffff - ((m.l[i - 1] >> 16) & 1);
            m.l[i - 1] &= 0xffff;
        }
        m.l[15] = t.l[15] - 0x7fff - ((m.l[14] >> 16) & 1);
        const int64_t borrow = (m.l[15] >> 16) & 1;
        m.l[14] &= 0xffff;
        fe_cswap(t, m, 1 - borrow);  // keep t - p when it did not borrow
    }
    for (int i = 0; i < 16; ++i) {
        out[2 * i] = uint8_t(t.l[i]);
        out[2 * i + 1] = uint8_t(t.l[i] >> 8);
    }
}

__device__ void x25519(uint8_t out[32], const uint8_t scalar[32], const uint8_t u[32])
{
    uint8_t k[32];
    for (int i = 0; i < 32; ++i) k[i] = scalar[i];
    k[0] &= 248;
    k[31] &= 127;
    k[31] |= 64;
    Fe x1, x2, z2, x3, z3, a, aa, b, bb, e, c, d, da, cb, t;
    fe_unpack(x1, u);
    for (int i = 0; i < 16; ++i) {
        x2.l[i] = z2.l[i] = z3.l[i] = 0;
        x3.l[i] = x1.l[i];
    }
    x2.l[0] = 1;
    z3.l[0] = 1;
    int64_t swap = 0;
    for (int pos = 254; pos >= 0; --pos) {
        const int64_t bit = (k[pos >> 3] >> (pos & 7)) & 1;
        swap ^= bit;
        fe_cswap(x2, x3, swap);
        fe_cswap(z2, z3, swap);
        swap = bit;
        fe_add(a, x2, z2);
        fe_mul(aa, a, a);
        fe_sub(b, x2, z2);
        fe_mul(bb, b, b);
        fe_sub(e, aa, bb);
        fe_add(c, x3, z3);
        fe_sub(d, x3, z3);
        fe_mul(da, d, a);
        fe_mul(cb, c, b);
        fe_add(t, da, cb);
        fe_mul(x3, t, t);
        fe_sub(t, da, cb);
        fe_mul(t, t, t);
        fe_mul(z3, x1, t);
        fe_mul(x2, aa, bb);
        fe_mul_small(t, e, 121665);
        fe_add(t, aa, t);
        fe_mul(z2, e, t);
    }
    fe_cswap(x2, x3, swap);
    fe_cswap(z2, z3, swap);
    fe_invert(z2, z2);
    fe_mul(x2, x2, z2);
    fe_pack(out, x2);
    for (int i = 0; i < 32; ++i) k[i] = 0;
}

// ---------------------------------------------------------------- kernels

constexpr char kInfo[] = "SecureInfer X25519 BLAKE2b test v1";

// Timing jitter of racing waves: every lane times contended atomic
// increments on one word and keeps the low bits of its clock readings.
__global__ void entropy_kernel(uint32_t* pool, uint32_t* counter, uint32_t rounds)
{
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (uint32_t i = 0; i < rounds; ++i) {
        const uint64_t t0 = clock64();
        const uint32_t old = atomicAdd(counter, 1u);
        const uint64_t t1 = clock64();
        acc = (acc << 5 | acc >> 27) ^ uint32_t(t1 - t0) ^ (old << 7) ^ uint32_t(wall_clock64());
    }
    pool[gid] = acc;
}

// Clears secret bytes in private memory through volatile stores, which the
// compiler cannot drop as dead.
__device__ void scrub(uint8_t* p, int n)
{
    volatile uint8_t* v = p;
    for (int i = 0; i < n; ++i) v[i] = 0;
}

// The device half of key_agreement.aicpu:9-49 with its status codes: 1 while
// the secret is drawn, 2 once it is (a zero shared secret stops there), 3
// while the key and proof are derived, 0 when done.  The device public value
// is written as soon as it is known, the key and the proof at the end.
__global__ void agree_kernel(const uint8_t* host_public, const uint8_t* challenge, AgreeSeed seed,
                             const uint32_t* pool, uint32_t pool_words, uint8_t* key_out,
                             uint8_t* device_public, uint8_t* proof_out, int32_t* status)
{
    if (threadIdx.x != 0) return;
    uint8_t secret[32], shared[32], base[32] = {9}, digest[64];
    *status = 1;
    B2b s;
    b2b_init(s, nullptr, 0, 64);
    b2b_update(s, seed.b, 32);
    b2b_update(s, reinterpret_cast<const uint8_t*>(pool), uint64_t(pool_words) * 4);
    b2b_final(s, digest);
    for (int i = 0; i < 32; ++i) secret[i] = digest[i];
    *status = 2;
    uint8_t dpub[32];
    x25519(dpub, secret, base);
    for (int i = 0; i < 32; ++i) device_public[i] = dpub[i];
    x25519(shared, secret, host_public);
    uint8_t nz = 0;
    for (int i = 0; i < 32; ++i) nz |= shared[i];
    if (!nz) {
        scrub(secret, 32);
        scrub(digest, 64);
        scrub(reinterpret_cast<uint8_t*>(&s), int(sizeof(s)));
        return;
    }
    *status = 3;
    uint8_t key[16], proof[32];
    b2b_init(s, shared, 32, 16);
    b2b_update(s, reinterpret_cast<const uint8_t*>(kInfo), sizeof(kInfo) - 1);
    b2b_update(s, host_public, 32);
    b2b_update(s, dpub, 32);
    b2b_update(s, challenge, 32);
    b2b_final(s, key);
    b2b_init(s, key, 16, 32);
    b2b_update(s, challenge, 32);
    b2b_final(s, proof);
    for (int i = 0; i < 16; ++i) key_out[i] = key[i];
    for (int i = 0; i < 32; ++i) proof_out[i] = proof[i];
    scrub(secret, 32);
    scrub(shared, 32);
    scrub(digest, 64);
    scrub(key, 16);
    scrub(reinterpret_cast<uint8_t*>(&s), int(sizeof(s)));
    __threadfence();
    *status = 0;
}

__device__ uint4 gf_one() { return make_uint4(0x80u, 0u, 0u, 0u); }

// H^e from the squarings sq[b] = H^(2^b).
__device__ uint4 gf_pow(const uint4* sq, uint32_t e)
{
    uint4 p = gf_one();
    for (int b = 0; b < 32; ++b)
        if ((e >> b) & 1) p = gf_mul4(p, sq[b]);
    return p;
}

// The record kernels' context from a device-resident key, in the host
// builder's layout: round keys, H, the powers H^0 .. H^(npow-1) and the
// 4-bit tables (32 nibble positions x 16 values) of H^T, H^2T, H^UT, H^2UT.
// One workgroup of 256 threads; te0 (public) is given.
__global__ __launch_bounds__(256) void ctx_build_kernel(const uint8_t* key, const uint32_t* te0, GcmCtx* c,
                                                        uint32_t npow)
{
    __shared__ uint8_t sbox[256];
    __shared__ uint32_t rk[44];
    __shared__ uint4 sq[32];
    __shared__ uint4 mult[4];
    const uint32_t tid = threadIdx.x;
    c->te0[tid] = te0[tid];
    sbox[tid] = uint8_t(te0[tid] >> 8);
    __syncthreads();
    if (tid == 0) {
        // AES-128 key expansion (FIPS-197 5.2), words as little-endian columns
        for (int i = 0; i < 4; ++i)
            rk[i] = uint32_t(key[4 * i]) | uint32_t(key[4 * i + 1]) << 8 | uint32_t(key[4 * i + 2]) << 16 |
                    uint32_t(key[4 * i + 3]) << 24;
        uint8_t rcon = 1;
        for (int i = 4; i < 44; ++i) {
            uint32_t t = rk[i - 1];
            if (i % 4 == 0) {
                t = (t >> 8) | (t << 24);  // RotWord on little-endian bytes
                t = uint32_t(sbox[t & 0xff]) | uint32_t(sbox[(t >> 8) & 0xff]) << 8 |
                    uint32_t(sbox[(t >> 16) & 0xff]) << 16 | uint32_t(sbox[t >> 24]) << 24;
                t ^= rcon;
                rcon = uint8_t((rcon << 1) ^ ((rcon & 0x80) ? 0x1b : 0));
            }
            rk[i] = rk[i - 4] ^ t;
        }
        // H = E_K(0^128) with byte-wise rounds
        uint8_t st[16];
        for (int i = 0; i < 16; ++i) st[i] = uint8_t(rk[i >> 2] >> (8 * (i & 3)));
        for (int r = 1; r <= 10; ++r) {
            uint8_t t[16];
            for (int i = 0; i < 16; ++i) t[i] = sbox[st[(i + 4 * (i & 3)) & 15]];  // SubBytes + ShiftRows
            if (r < 10) {
                for (int col = 0; col < 4; ++col) {  // MixColumns
                    const uint8_t* a = t + 4 * col;
                    uint8_t m[4];
                    for (int j = 0; j < 4; ++j) {
                        const uint8_t x = a[j], y = a[(j + 1) & 3];
                        const uint8_t x2 = uint8_t((x << 1) ^ ((x & 0x80) ? 0x1b : 0));
                        const uint8_t y2 = uint8_t((y << 1) ^ ((y & 0x80) ? 0x1b : 0));
                        m[j] = uint8_t(x2 ^ y2 ^ y ^ a[(j + 2) & 3] ^ a[(j + 3) & 3]);
                    }
                    for (int j = 0; j < 4; ++j) st[4 * col + j] = m[j];
                }
            } else {
                for (int i = 0; i < 16; ++i) st[i] = t[i];
            }
            for (int i = 0; i < 16; ++i) st[i] ^= uint8_t(rk[4 * r + (i >> 2)] >> (8 * (i & 3)));
        }
        uint32_t hw[4];
        for (int k = 0; k < 4; ++k)
            hw[k] = uint32_t(st[4 * k]) | uint32_t(st[4 * k + 1]) << 8 | uint32_t(st[4 * k + 2]) << 16 |
                    uint32_t(st[4 * k + 3]) << 24;
        sq[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        for (int b = 1; b < 32; ++b) sq[b] = gf_mul4(sq[b - 1], sq[b - 1]);
        mult[0] = gf_pow(sq, SI_T);
        mult[1] = gf_pow(sq, 2 * SI_T);
        mult[2] = gf_pow(sq, SI_U * SI_T);
        mult[3] = gf_pow(sq, 2 * SI_U * SI_T);
    }
    __syncthreads();
    if (tid < 44) {
        c->rk[tid] = rk[tid];
        c->rk16[tid] = (rk[tid] << 16) | (rk[tid] >> 16);
    }
    if (tid == 0) {
        c->h[0] = sq[0].x;
        c->h[1] = sq[0].y;
        c->h[2] = sq[0].z;
        c->h[3] = sq[0].w;
        c->npow = npow;
        c->reserved[0] = c->reserved[1] = c->reserved[2] = 0;
    }
    // Powers: thread t starts at H^t and steps by H^256.
    uint4* pow = reinterpret_cast<uint4*>(c + 1);
    if (tid < npow) {
        uint4 p = gf_pow(sq, tid);
        for (uint32_t e = tid; e < npow; e += 256) {
            pow[e] = p;
            p = gf_mul4(p, sq[8]);
        }
    }
    // Tables: entry (pos, v) of multiplier m = m * x, x zero except byte
    // pos / 2, which holds v (even pos) or v << 4 (odd pos).
    uint4* tbl[4] = {c->gh4, c->gh4b, c->gh4u, c->gh4u2};
    for (uint32_t i = tid; i < 4 * 512; i += 256) {
        const uint32_t t = i >> 9, pos = (i >> 4) & 31, v = i & 15;
        const uint32_t byte = (pos & 1) ? v << 4 : v;
        uint32_t xw[4] = {0, 0, 0, 0};
        xw[(pos >> 1) >> 2] = byte << (8 * ((pos >> 1) & 3));
        tbl[t][pos * 16 + v] = gf_mul4(make_uint4(xw[0], xw[1], xw[2], xw[3]), mult[t]);
    }
}

// Single-lane runs of the device X25519 and BLAKE2b for the tests.
__global__ void x25519_test_kernel(const uint8_t* scalar, const uint8_t* u, uint8_t* out)
{
    if (threadIdx.x == 0) x25519(out, scalar, u);
}

__global__ void blake2b_test_kernel(const uint8_t* key, uint32_t key_len, const uint8_t* msg, uint64_t msg_len,
                                    uint8_t* out, uint32_t out_len)
{
    if (threadIdx.x != 0) return;
    B2b s;
    b2b_init(s, key, key_len, out_len);
    b2b_update(s, msg, msg_len);
    b2b_final(s, out);
}

__global__ void zero_bytes_kernel(uint8_t* p, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t launch_agree(hipStream_t stream, const uint8_t* host_public, const uint8_t* challenge,
                        const AgreeSeed& seed, uint32_t* pool, uint32_t* counter, uint8_t* key_out,
                        uint8_t* device_public, uint8_t* proof, int32_t* status)
{
    constexpr uint32_t kBlocks = 512, kThreads = 256, kRounds = 8;
    static_assert(kBlocks * kThreads == SI_AGREE_POOL_WORDS, "pool size");
    hipLaunchKernelGGL(zero_bytes_kernel, dim3(1), dim3(64), 0, stream, reinterpret_cast<uint8_t*>(counter), 4u);
    hipLaunchKernelGGL(entropy_kernel, dim3(kBlocks), dim3(kThreads), 0, stream, pool, counter, kRounds);
    hipLaunchKernelGGL(agree_kernel, dim3(1), dim3(64), 0, stream, host_public, challenge, seed, pool,
                       kBlocks * kThreads, key_out, device_public, proof, status);
    return hipGetLastError();
}

hipError_t launch_ctx_build(hipStream_t stream, const uint8_t* key, const uint32_t* te0, GcmCtx* ctx,
                            uint32_t npow)
{
    hipLaunchKernelGGL(ctx_build_kernel, dim3(1), dim3(256), 0, stream, key, te0, ctx, npow);
    return hipGetLastError();
}

hipError_t launch_zero_bytes(hipStream_t stream, uint8_t* p, uint32_t n)
{
    hipLaunchKernelGGL(zero_bytes_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

hipError_t launch_x25519_test(hipStream_t stream, const uint8_t* scalar, const uint8_t* u, uint8_t* out)
{
    hipLaunchKernelGGL(x25519_test_kernel, dim3(1), dim3(64), 0, stream, scalar, u, out);
    return hipGetLastError();
}

hipError_t launch_blake2b_test(hipStream_t stream, const uint8_t* key, uint32_t key_len, const uint8_t* msg,
                               uint64_t msg_len, uint8_t* out, uint32_t out_len)
{
    hipLaunchKernelGGL(blake2b_test_kernel, dim3(1), dim3(64), 0, stream, key, key_len, msg, msg_len, out, out_len);
    return hipGetLastError();
}

}  // namespace si
