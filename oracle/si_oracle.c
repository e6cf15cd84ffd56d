/*
 * CPU oracle for the authenticated KV reload / writeback path.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, to check results against.  The product library never
 * links or calls it.
 *
 * Written from the specifications (FIPS-197, NIST SP 800-38D) and from the
 * reference call sites cited per function.  Built with -ffp-contract=off so
 * the codec's float32 arithmetic keeps one rounding per torch operation.
 */
#include "si_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* AES-128, FIPS-197.  The S-box is derived, not tabulated: multiplicative
 * inverse in GF(2^8) mod x^8+x^4+x^3+x+1 followed by the affine map
 * b ^ rotl(b,1..4) ^ 0x63 (FIPS-197 5.1.1).  The reference kernel's key
 * schedule and round structure are ghash.aicpu:60-131.                   */

static uint8_t g_sbox[256];
static int g_sbox_ready;

static uint8_t gf8_mul(uint8_t a, uint8_t b)
{
    uint8_t r = 0;
    while (b) {
        if (b & 1) r ^= a;
        a = (uint8_t)((a << 1) ^ ((a & 0x80) ? 0x1b : 0));
        b >>= 1;
    }
    return r;
}

static uint8_t rotl8(uint8_t x, int s) { return (uint8_t)((x << s) | (x >> (8 - s))); }

static void build_sbox(void)
{
    if (g_sbox_ready) return;
    for (int x = 0; x < 256; ++x) {
        uint8_t inv = 0;
        if (x) {
            /* x^254 = x^-1 in GF(2^8) */
            uint8_t p = (uint8_t)x, acc = 1;
            int e = 254;
            while (e) {
                if (e & 1) acc = gf8_mul(acc, p);
                p = gf8_mul(p, p);
                e >>= 1;
            }
            inv = acc;
        }
        g_sbox[x] = (uint8_t)(inv ^ rotl8(inv, 1) ^ rotl8(inv, 2) ^ rotl8(inv, 3) ^
                              rotl8(inv, 4) ^ 0x63);
    }
    g_sbox_ready = 1;
}

void si_or_sbox(uint8_t out[256])
{
    build_sbox();
    memcpy(out, g_sbox, 256);
}

void si_or_aes128_expand(const uint8_t key[16], uint8_t rk[176])
{
    build_sbox();
    memcpy(rk, key, 16);
    uint8_t rcon = 1;
    for (int i = 4; i < 44; ++i) {
        uint8_t t[4];
        memcpy(t, rk + 4 * (i - 1), 4);
        if (i % 4 == 0) {
            uint8_t f = t[0];
            t[0] = (uint8_t)(g_sbox[t[1]] ^ rcon);
            t[1] = g_sbox[t[2]];
            t[2] = g_sbox[t[3]];
            t[3] = g_sbox[f];
            rcon = gf8_mul(rcon, 2);
        }
        for (int j = 0; j < 4; ++j) rk[4 * i + j] = (uint8_t)(rk[4 * (i - 4) + j] ^ t[j]);
    }
}

void si_or_aes128_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16])
{
    build_sbox();
    uint8_t s[16], t[16];
    for (int i = 0; i < 16; ++i) s[i] = (uint8_t)(in[i] ^ rk[i]);
    for (int round = 1; round <= 10; ++round) {
        /* SubBytes + ShiftRows: state byte (row r, col c) is s[r + 4c]. */
        for (int c = 0; c < 4; ++c)
            for (int r = 0; r < 4; ++r) t[r + 4 * c] = g_sbox[s[r + 4 * ((c + r) & 3)]];
        if (round != 10) {
            for (int c = 0; c < 4; ++c) {
                uint8_t a0 = t[4 * c], a1 = t[4 * c + 1], a2 = t[4 * c + 2], a3 = t[4 * c + 3];
                s[4 * c + 0] = (uint8_t)(gf8_mul(a0, 2) ^ gf8_mul(a1, 3) ^ a2 ^ a3);
                s[4 * c + 1] = (uint8_t)(a0 ^ gf8_mul(a1, 2) ^ gf8_mul(a2, 3) ^ a3);
                s[4 * c + 2] = (uint8_t)(a0 ^ a1 ^ gf8_mul(a2, 2) ^ gf8_mul(a3, 3));
                s[4 * c + 3] = (uint8_t)(gf8_mul(a0, 3) ^ a1 ^ a2 ^ gf8_mul(a3, 2));
            }
        } else {
            memcpy(s, t, 16);
        }
        for (int i = 0; i < 16; ++i) s[i] ^= rk[16 * round + i];
    }
    memcpy(out, s, 16);
}

/* ------------------------------------------------------------------ */
/* GF(2^128) multiply, SP 800-38D Algorithm 1.  Bit 0 of a block is the MSB
 * of byte 0; R = 11100001 || 0^120.                                     */

void si_or_gf128_mul(const uint8_t x[16], const uint8_t y[16], uint8_t z[16])
{
    uint8_t v[16], r[16] = {0};
    memcpy(v, y, 16);
    for (int i = 0; i < 128; ++i) {
        if ((x[i >> 3] >> (7 - (i & 7))) & 1)
            for (int k = 0; k < 16; ++k) r[k] ^= v[k];
        int lsb = v[15] & 1;
        for (int k = 15; k > 0; --k) v[k] = (uint8_t)((v[k] >> 1) | (v[k - 1] << 7));
        v[0] >>= 1;
        if (lsb) v[0] ^= 0xe1;
    }
    memcpy(z, r, 16);
}

static void ghash_update(const uint8_t h[16], uint8_t s[16], const uint8_t* data, uint64_t bytes)
{
    /* Each input is zero-padded to a 16-byte multiple on its own
     * (ghash.aicpu:338-496 pads the AAD and the ciphertext separately). */
    for (uint64_t off = 0; off < bytes; off += 16) {
        uint8_t blk[16] = {0};
        uint64_t take = bytes - off < 16 ? bytes - off : 16;
        memcpy(blk, data + off, (size_t)take);
        for (int k = 0; k < 16; ++k) s[k] ^= blk[k];
        si_or_gf128_mul(s, h, s);
    }
}

static void store_be64(uint8_t* out, uint64_t v)
{
    for (int i = 0; i < 8; ++i) out[i] = (uint8_t)(v >> (56 - 8 * i));
}

static void store_be32(uint8_t* out, uint32_t v)
{
    for (int i = 0; i < 4; ++i) out[i] = (uint8_t)(v >> (24 - 8 * i));
}

void si_or_ghash(const uint8_t h[16], const uint8_t* aad, uint64_t aad_bytes,
                 const uint8_t* data, uint64_t bytes, uint8_t s[16])
{
    /* S = GHASH_H(A || 0^v || C || 0^u || [len(A)]_64 || [len(C)]_64)
     * (ghash.aicpu:623-634, length block from store_be64 :508-513). */
    memset(s, 0, 16);
    if (aad_bytes) ghash_update(h, s, aad, aad_bytes);
    ghash_update(h, s, data, bytes);
    uint8_t len[16];
    store_be64(len, aad_bytes * 8);
    store_be64(len + 8, bytes * 8);
    for (int k = 0; k < 16; ++k) s[k] ^= len[k];
    si_or_gf128_mul(s, h, s);
}

/* ------------------------------------------------------------------ */
/* CTR: counter block = BE(iv0) BE(iv1) BE(iv2) BE32(counter), counter starts
 * at iv_words[3] and wraps in 32 bits (make_counter_block and
 * aes128_ctr_process, ghash.aicpu:133-147, 174-221).                      */

static void counter_block(const uint32_t iv[4], uint32_t ctr, uint8_t out[16])
{
    for (int w = 0; w < 3; ++w) store_be32(out + 4 * w, iv[w]);
    store_be32(out + 12, ctr);
}

void si_or_keystream(const uint8_t key[16], const uint32_t iv_words[4], uint8_t* out,
                     uint64_t bytes)
{
    uint8_t rk[176], cb[16], ks[16];
    si_or_aes128_expand(key, rk);
    uint32_t ctr = iv_words[3];
    for (uint64_t off = 0; off < bytes; off += 16, ++ctr) {
        counter_block(iv_words, ctr, cb);
        si_or_aes128_encrypt(rk, cb, ks);
        uint64_t take = bytes - off < 16 ? bytes - off : 16;
        memcpy(out + off, ks, (size_t)take);
    }
}

void si_or_aes_ctr(const uint8_t key[16], const uint32_t iv_words[4], const uint8_t* in,
                   uint8_t* out, uint64_t bytes)
{
    uint8_t rk[176], cb[16], ks[16];
    si_or_aes128_expand(key, rk);
    uint32_t ctr = iv_words[3];
    for (uint64_t off = 0; off < bytes; off += 16, ++ctr) {
        counter_block(iv_words, ctr, cb);
        si_or_aes128_encrypt(rk, cb, ks);
        uint64_t take = bytes - off < 16 ? bytes - off : 16;
        for (uint64_t k = 0; k < take; ++k) out[off + k] = (uint8_t)(in[off + k] ^ ks[k]);
    }
}

static void tag_mask(const uint8_t key[16], const uint32_t iv_words[4], uint8_t mask[16])
{
    /* E_K(J0) with J0 = nonce || 1 (ghash.aicpu:615-620). */
    uint8_t rk[176], j0[16];
    si_or_aes128_expand(key, rk);
    counter_block(iv_words, 1u, j0);
    si_or_aes128_encrypt(rk, j0, mask);
}

void si_or_gcm_encrypt_tag(const uint8_t key[16], const uint8_t h[16],
                           const uint32_t iv_words[4], const uint8_t* aad,
                           uint64_t aad_bytes, const uint8_t* pt, uint64_t bytes,
                           uint8_t* ct, uint8_t tag[16])
{
    /* secure_infer_gcm_encrypt_tag, ghash.aicpu:656-699 */
    uint8_t s[16], m[16];
    si_or_aes_ctr(key, iv_words, pt, ct, bytes);
    si_or_ghash(h, aad, aad_bytes, ct, bytes, s);
    tag_mask(key, iv_words, m);
    for (int k = 0; k < 16; ++k) tag[k] = (uint8_t)(s[k] ^ m[k]);
}

uint32_t si_or_gcm_decrypt_verify(const uint8_t key[16], const uint8_t h[16],
                                  const uint32_t iv_words[4], const uint8_t* aad,
                                  uint64_t aad_bytes, const uint8_t* ct,
                                  uint64_t bytes, const uint8_t expected_tag[16],
                                  uint8_t* out)
{
    /* secure_infer_gcm_decrypt_verify, ghash.aicpu:594-651: constant-time
     * OR-reduce compare, CTR decrypt, AND-mask the output with 0x00/0xff. */
    uint8_t s[16], m[16], diff = 0;
    si_or_ghash(h, aad, aad_bytes, ct, bytes, s);
    tag_mask(key, iv_words, m);
    for (int k = 0; k < 16; ++k) diff |= (uint8_t)(s[k] ^ m[k] ^ expected_tag[k]);
    uint32_t ok = diff == 0 ? 1u : 0u;
    si_or_aes_ctr(key, iv_words, ct, out, bytes);
    uint8_t mask = (uint8_t)(0u - ok);
    for (uint64_t i = 0; i < bytes; ++i) out[i] &= mask;
    return ok;
}

/* ------------------------------------------------------------------ */
/* Ticket / IV / AAD                                                     */

void si_or_derive_transfer_iv(const uint8_t base_iv[16], uint64_t session_nonce,
                              uint64_t ticket, uint64_t block_offset, uint8_t out_iv[16])
{
    /* secure_infer_derive_transfer_iv, secure_infer.cpp:274-300 (GCM:
     * counter_base 2; bytes 4..11 = BE64(session_nonce + ticket)). */
    memcpy(out_iv, base_iv, 16);
    store_be64(out_iv + 4, session_nonce + ticket);
    store_be32(out_iv + 12, (uint32_t)(block_offset + 2));
}

void si_or_pack_iv_words(const uint8_t iv[16], uint32_t words[4])
{
    /* pack_inline_iv, secure_infer.cpp:2083-2093 */
    for (int w = 0; w < 4; ++w)
        words[w] = ((uint32_t)iv[4 * w] << 24) | ((uint32_t)iv[4 * w + 1] << 16) |
                   ((uint32_t)iv[4 * w + 2] << 8) | (uint32_t)iv[4 * w + 3];
}

void si_or_build_gcm_aad(uint8_t direction, uint32_t tensor_kind, uint32_t layer_id,
                         uint64_t block_id, uint64_t byte_offset, uint64_t bytes,
                         uint64_t ticket, uint64_t transfer_offset,
                         uint64_t session_nonce, uint8_t out[64])
{
    /* secure_infer_build_gcm_aad, secure_infer.cpp:730-775 */
    memset(out, 0, 64);
    out[0] = 'S'; out[1] = 'F'; out[2] = 'A'; out[3] = 'D';
    out[4] = 1;
    out[5] = direction;
    out[6] = (uint8_t)(tensor_kind & 0xff);
    store_be32(out + 8, layer_id);
    store_be64(out + 12, block_id);
    store_be64(out + 20, byte_offset);
    store_be64(out + 28, bytes);
    store_be64(out + 36, ticket);
    store_be64(out + 44, transfer_offset);
    store_be64(out + 52, session_nonce);
}

/* ------------------------------------------------------------------ */
/* KV codec.  One record = one 128-token block of one kind, [128, h, d].
 * transport_codec.py:22-42 (encode), optimized_decode.py:5-26 (decode).   */

#define SI_TOKENS 128u
#define SI_GROUP 64u

uint64_t si_or_codec_qbytes(uint32_t bits, uint32_t heads, uint32_t dim)
{
    return (uint64_t)SI_TOKENS * heads * dim * bits / 8u;
}

uint64_t si_or_codec_sbytes(uint32_t heads, uint32_t dim)
{
    /* K: (t/64, h, d) params; V: (t, h, d/64) params -> both 2*h*d floats */
    return (uint64_t)(SI_TOKENS / SI_GROUP) * heads * dim * 4u;
}

uint64_t si_or_codec_width(uint32_t bits, uint32_t heads, uint32_t dim)
{
    uint64_t w = si_or_codec_qbytes(bits, heads, dim) + 2 * si_or_codec_sbytes(heads, dim) + 16;
    return (w + 15) / 16 * 16;
}

static float bf16_to_f32(uint16_t v)
{
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t si_or_f32_to_bf16(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* parameter index of element (t, hh, dd) */
static uint64_t param_index(uint32_t kind, uint32_t heads, uint32_t dim, uint32_t t,
                            uint32_t hh, uint32_t dd)
{
    if (kind == 0) return ((uint64_t)(t / SI_GROUP) * heads + hh) * dim + dd;
    return ((uint64_t)t * heads + hh) * (dim / SI_GROUP) + dd / SI_GROUP;
}

/* x.amin / x.amax as torch computes them for a group: a NaN anywhere makes
 * the result NaN (transport_codec.py:30-31); equal zeros order -0 < +0
 * (IEEE 754-2019 minimum / maximum).  lo/hi start at +inf / -inf.        */
static void minmax_update(float x, float* lo, float* hi)
{
    if (isnan(*lo)) return;
    if (isnan(x)) { *lo = x; *hi = x; return; }
    if (x < *lo || (x == *lo && signbit(x) && !signbit(*lo))) *lo = x;
    if (x > *hi || (x == *hi && !signbit(x) && signbit(*hi))) *hi = x;
}

void si_or_codec_encode(const uint16_t* block_bf16, uint32_t heads, uint32_t dim,
                        uint32_t bits, uint32_t kind, uint32_t layer, uint8_t* packet)
{
    const uint64_t hd = (uint64_t)heads * dim;
    const uint64_t n = SI_TOKENS * hd;
    const uint64_t np = si_or_codec_sbytes(heads, dim) / 4;
    const uint64_t qb = si_or_codec_qbytes(bits, heads, dim);
    const uint64_t sb = np * 4;
    const uint64_t width = si_or_codec_width(bits, heads, dim);
    const float qmax = (float)((1u << bits) - 1u);
    memset(packet, 0, (size_t)width);
    float* lo = (float*)malloc((size_t)np * sizeof(float));
    float* hi = (float*)malloc((size_t)np * sizeof(float));
    float* scale = (float*)malloc((size_t)np * sizeof(float));
    for (uint64_t p = 0; p < np; ++p) { lo[p] = INFINITY; hi[p] = -INFINITY; }
    /* x.amin / x.amax over the group axis: tokens for K, dims for V. */
    for (uint32_t t = 0; t < SI_TOKENS; ++t)
        for (uint32_t hh = 0; hh < heads; ++hh)
            for (uint32_t dd = 0; dd < dim; ++dd) {
                float x = bf16_to_f32(block_bf16[(uint64_t)t * hd + (uint64_t)hh * dim + dd]);
                uint64_t p = param_index(kind, heads, dim, t, hh, dd);
                minmax_update(x, &lo[p], &hi[p]);
            }
    /* scale = ((high-low)/(2^bits-1)).clamp_min(1e-12), float32 throughout */
    const float floor_scale = 1e-12f;
    for (uint64_t p = 0; p < np; ++p) {
        volatile float diff = hi[p] - lo[p];
        volatile float s = diff / qmax;
        scale[p] = s < floor_scale ? floor_scale : s;
    }
    /* q = ((x-low)/scale).round().clamp(0, 2^bits-1), flattened (t, h, d);
     * int4 then packs q[2j] + 16*q[2j+1] in float (a NaN in either element
     * makes the byte's value NaN) before the uint8 cast. */
    float qpair = 0.0f;
    for (uint64_t e = 0; e < n; ++e) {
        uint32_t t = (uint32_t)(e / hd);
        uint32_t hh = (uint32_t)((e % hd) / dim);
        uint32_t dd = (uint32_t)(e % dim);
        uint64_t p = param_index(kind, heads, dim, t, hh, dd);
        float x = bf16_to_f32(block_bf16[e]);
        volatile float num = x - lo[p];
        volatile float r = num / scale[p];
        float q = rintf(r);
        if (q < 0.0f) q = 0.0f;
        if (q > qmax) q = qmax;
        /* round().clamp() keeps NaN; torch's float -> uint8 cast then gives 0
         * (the x86 conversion yields 0x80000000, whose low byte is 0). */
        if (bits == 8) {
            packet[e] = isnan(q) ? 0u : (uint8_t)(uint32_t)q;
        } else if ((e & 1) == 0) {
            qpair = q;
        } else {
            volatile float v = qpair + 16.0f * q;
            packet[e >> 1] = isnan(v) ? 0u : (uint8_t)(uint32_t)v;
        }
    }
    memcpy(packet + qb, scale, (size_t)sb);
    memcpy(packet + qb + sb, lo, (size_t)sb);
    int32_t header[4] = {1, (int32_t)layer, (int32_t)kind, (int32_t)bits};
    memcpy(packet + qb + 2 * sb, header, 16);
    free(lo);
    free(hi);
    free(scale);
}

void si_or_codec_decode(const uint8_t* packet, uint32_t heads, uint32_t dim,
                        uint32_t bits, uint32_t kind, uint16_t* block_bf16)
{
    const uint64_t hd = (uint64_t)heads * dim;
    const uint64_t n = SI_TOKENS * hd;
    const uint64_t qb = si_or_codec_qbytes(bits, heads, dim);
    const uint64_t sb = si_or_codec_sbytes(heads, dim);
    for (uint64_t e = 0; e < n; ++e) {
        uint32_t t = (uint32_t)(e / hd);
        uint32_t hh = (uint32_t)((e % hd) / dim);
        uint32_t dd = (uint32_t)(e % dim);
        uint64_t p = param_index(kind, heads, dim, t, hh, dd);
        float q;
        if (bits == 8) {
            q = (float)packet[e];
        } else {
            /* high = floor(p/16), low = p - 16*high; element 2j = low nibble */
            uint8_t b = packet[e >> 1];
            q = (float)((e & 1) ? (b >> 4) : (b & 15));
        }
        float s, o;
        memcpy(&s, packet + qb + 4 * p, 4);
        memcpy(&o, packet + qb + sb + 4 * p, 4);
        /* values.mul_(scale); values.add_(offset): two float32 roundings */
        volatile float v = q * s;
        volatile float w = v + o;
        block_bf16[e] = si_or_f32_to_bf16(w);
    }
}
