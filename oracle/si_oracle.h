/*
 * CPU oracle for the authenticated KV reload / writeback path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only to check results against.
 *
 * Every function restates the reference algorithm from its specification and
 * cites the reference call site it follows:
 *   AES-128            FIPS-197 (S-box derived from GF(2^8) inversion + affine map)
 *   GHASH / GCM        NIST SP 800-38D, Algorithm 1 (bit-serial multiply)
 *   IV / AAD / ticket  secure_infer/native/secure_infer.cpp:261-300, 730-775
 *   device GCM kernels secure_infer/native/kernels/aicpu/ghash.aicpu:133-147,
 *                      594-699, 1051-1068
 *   KV codec           secure_infer/kv_offload/transport_codec.py:22-42,
 *                      secure_infer/kv_offload/optimized_decode.py:5-26
 */
#ifndef SI_ORACLE_H
#define SI_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- AES-128 (FIPS-197) ---- */
void si_or_aes128_expand(const uint8_t key[16], uint8_t rk[176]);
void si_or_aes128_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]);
void si_or_sbox(uint8_t out[256]);

/* ---- GF(2^128) and GHASH (SP 800-38D) ---- */
void si_or_gf128_mul(const uint8_t x[16], const uint8_t y[16], uint8_t z[16]);
void si_or_ghash(const uint8_t h[16], const uint8_t* aad, uint64_t aad_bytes,
                 const uint8_t* data, uint64_t bytes, uint8_t s[16]);

/* ---- CTR and GCM in the reference kernel ABI form (iv_words = 4 BE u32) ---- */
void si_or_keystream(const uint8_t key[16], const uint32_t iv_words[4],
                     uint8_t* out, uint64_t bytes);
void si_or_aes_ctr(const uint8_t key[16], const uint32_t iv_words[4],
                   const uint8_t* in, uint8_t* out, uint64_t bytes);
void si_or_gcm_encrypt_tag(const uint8_t key[16], const uint8_t h[16],
                           const uint32_t iv_words[4], const uint8_t* aad,
                           uint64_t aad_bytes, const uint8_t* pt, uint64_t bytes,
                           uint8_t* ct, uint8_t tag[16]);
uint32_t si_or_gcm_decrypt_verify(const uint8_t key[16], const uint8_t h[16],
                                  const uint32_t iv_words[4], const uint8_t* aad,
                                  uint64_t aad_bytes, const uint8_t* ct,
                                  uint64_t bytes, const uint8_t expected_tag[16],
                                  uint8_t* out);

/* ---- ticket / IV / AAD (secure_infer.cpp) ---- */
void si_or_derive_transfer_iv(const uint8_t base_iv[16], uint64_t session_nonce,
                              uint64_t ticket, uint64_t block_offset,
                              uint8_t out_iv[16]);
void si_or_pack_iv_words(const uint8_t iv[16], uint32_t words[4]);
void si_or_build_gcm_aad(uint8_t direction, uint32_t tensor_kind, uint32_t layer_id,
                         uint64_t block_id, uint64_t byte_offset, uint64_t bytes,
                         uint64_t ticket, uint64_t transfer_offset,
                         uint64_t session_nonce, uint8_t out[64]);

/* ---- KV codec (transport_codec.encode / optimized_decode.decode_into) ---- */
uint64_t si_or_codec_qbytes(uint32_t bits, uint32_t heads, uint32_t dim);
uint64_t si_or_codec_sbytes(uint32_t heads, uint32_t dim);
uint64_t si_or_codec_width(uint32_t bits, uint32_t heads, uint32_t dim);
void si_or_codec_encode(const uint16_t* block_bf16, uint32_t heads, uint32_t dim,
                        uint32_t bits, uint32_t kind, uint32_t layer,
                        uint8_t* packet);
void si_or_codec_decode(const uint8_t* packet, uint32_t heads, uint32_t dim,
                        uint32_t bits, uint32_t kind, uint16_t* block_bf16);
uint16_t si_or_f32_to_bf16(float x);

#ifdef __cplusplus
}
#endif
#endif
