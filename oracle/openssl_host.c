/*
 * Host-side AES-128-GCM through OpenSSL EVP, exactly as the reference's host
 * half calls it, plus a multi-threaded layer reload / writeback driver used
 * as the CPU baseline.
 *
 * TEST INFRASTRUCTURE ONLY: tests use it to pin the oracle (and the GPU path)
 * to OpenSSL's ciphertexts and tags; bench.py's cpu_baseline leg times it.
 *
 *   encrypt: inline_h2d_encrypt_commit, secure_infer.cpp:6486-6550
 *            (EVP_aes_128_gcm, IVLEN 12, 64-B AAD, 16-B tag)
 *   decrypt: d2h_host_decrypt_one, secure_infer.cpp:2470-2547
 *            (DecryptUpdate + SET_TAG + DecryptFinal; failure -> zero output)
 */
#include <openssl/evp.h>
#include <openssl/opensslv.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "si_oracle.h"

const char* si_ossl_version(void) { return OPENSSL_VERSION_TEXT; }

static int gcm_encrypt_ctx(EVP_CIPHER_CTX* ctx, const uint8_t* key, const uint8_t* iv12,
                           const uint8_t* aad, int aad_len, const uint8_t* pt, int n,
                           uint8_t* ct, uint8_t* tag)
{
    int len = 0, fin = 0;
    if (EVP_EncryptInit_ex(ctx, EVP_aes_128_gcm(), NULL, NULL, NULL) != 1) return -1;
    if (EVP_CIPHER_CTX_ctrl(ctx, EVP_CTRL_GCM_SET_IVLEN, 12, NULL) != 1) return -1;
    if (EVP_EncryptInit_ex(ctx, NULL, NULL, key, iv12) != 1) return -1;
    if (aad_len && EVP_EncryptUpdate(ctx, NULL, &len, aad, aad_len) != 1) return -1;
    if (n && EVP_EncryptUpdate(ctx, ct, &len, pt, n) != 1) return -1;
    if (EVP_EncryptFinal_ex(ctx, ct + len, &fin) != 1) return -1;
    if (EVP_CIPHER_CTX_ctrl(ctx, EVP_CTRL_GCM_GET_TAG, 16, tag) != 1) return -1;
    return 0;
}

static int gcm_decrypt_ctx(EVP_CIPHER_CTX* ctx, const uint8_t* key, const uint8_t* iv12,
                           const uint8_t* aad, int aad_len, const uint8_t* ct, int n,
                           const uint8_t* tag, uint8_t* pt)
{
    int len = 0, fin = 0, ok;
    ok = EVP_DecryptInit_ex(ctx, EVP_aes_128_gcm(), NULL, NULL, NULL) == 1 &&
         EVP_CIPHER_CTX_ctrl(ctx, EVP_CTRL_GCM_SET_IVLEN, 12, NULL) == 1 &&
         EVP_DecryptInit_ex(ctx, NULL, NULL, key, iv12) == 1;
    if (ok && aad_len) ok = EVP_DecryptUpdate(ctx, NULL, &len, aad, aad_len) == 1;
    if (ok && n) ok = EVP_DecryptUpdate(ctx, pt, &len, ct, n) == 1;
    if (ok)
        ok = EVP_CIPHER_CTX_ctrl(ctx, EVP_CTRL_GCM_SET_TAG, 16, (void*)tag) == 1 &&
             EVP_DecryptFinal_ex(ctx, pt + len, &fin) == 1;
    if (!ok && n) memset(pt, 0, (size_t)n);
    return ok ? 1 : 0;
}

int si_ossl_gcm_encrypt(const uint8_t key[16], const uint8_t iv12[12], const uint8_t* aad,
                        uint64_t aad_len, const uint8_t* pt, uint64_t n, uint8_t* ct,
                        uint8_t tag[16])
{
    EVP_CIPHER_CTX* ctx = EVP_CIPHER_CTX_new();
    if (!ctx) return -1;
    int rc = gcm_encrypt_ctx(ctx, key, iv12, aad, (int)aad_len, pt, (int)n, ct, tag);
    EVP_CIPHER_CTX_free(ctx);
    return rc;
}

int si_ossl_gcm_decrypt(const uint8_t key[16], const uint8_t iv12[12], const uint8_t* aad,
                        uint64_t aad_len, const uint8_t* ct, uint64_t n,
                        const uint8_t tag[16], uint8_t* pt)
{
    EVP_CIPHER_CTX* ctx = EVP_CIPHER_CTX_new();
    if (!ctx) return -1;
    int rc = gcm_decrypt_ctx(ctx, key, iv12, aad, (int)aad_len, ct, (int)n, tag, pt);
    EVP_CIPHER_CTX_free(ctx);
    return rc;
}

/* ------------------------------------------------------------------ */
/* Layer drivers.  One record = one (block, kind) slice.  The wire buffer
 * holds nrec records of `stride` bytes each: [ct count][pad][tag 16][16][aad 64]
 * (the reference's H2D wire record, secure_infer.cpp:6379-6388).          */

typedef struct {
    int direction; /* 1 = reload (decrypt+verify+[decode]+scatter), 2 = writeback */
    const uint8_t* key;
    const uint8_t* iv12; /* nrec x 12 */
    uint8_t* wire;
    uint64_t stride, count, tag_off, aad_off;
    uint32_t nrec;
    uint8_t* cache[2];   /* host paged caches, K and V */
    uint64_t slot_bytes;
    const int64_t* slots; /* nrec slots */
    const uint32_t* kinds;
    uint32_t bits, heads, dim, layer;
    uint8_t* scratch;    /* per-thread packet scratch (codec) */
    uint32_t* status;
    uint32_t r0, r1;
} layer_job;

static void* layer_worker(void* arg)
{
    layer_job* j = (layer_job*)arg;
    EVP_CIPHER_CTX* ctx = EVP_CIPHER_CTX_new();
    for (uint32_t r = j->r0; r < j->r1; ++r) {
        uint8_t* rec = j->wire + (uint64_t)r * j->stride;
        uint8_t* slot = j->cache[j->kinds[r]] + (uint64_t)j->slots[r] * j->slot_bytes;
        if (j->direction == 1) {
            uint8_t* dst = j->bits ? j->scratch : slot;
            uint32_t ok = (uint32_t)gcm_decrypt_ctx(ctx, j->key, j->iv12 + 12 * r,
                                                    rec + j->aad_off, 64, rec, (int)j->count,
                                                    rec + j->tag_off, dst);
            if (j->bits) {
                if (ok)
                    si_or_codec_decode(dst, j->heads, j->dim, j->bits, j->kinds[r],
                                       (uint16_t*)slot);
                else
                    memset(slot, 0, (size_t)j->slot_bytes);
            }
            j->status[r] = ok;
        } else {
            const uint8_t* src = slot;
            if (j->bits) {
                si_or_codec_encode((const uint16_t*)slot, j->heads, j->dim, j->bits,
                                   j->kinds[r], j->layer, j->scratch);
                src = j->scratch;
            }
            gcm_encrypt_ctx(ctx, j->key, j->iv12 + 12 * r, rec + j->aad_off, 64, src,
                            (int)j->count, rec, rec + j->tag_off);
        }
    }
    EVP_CIPHER_CTX_free(ctx);
    return NULL;
}

/* Runs the layer job with `threads` threads on a static record partition and
 * returns the wall time in nanoseconds.  The wire buffer is updated in place
 * for writeback; statuses are written for reload. */
int64_t si_ossl_layer(int direction, const uint8_t key[16], const uint8_t* iv12,
                      uint8_t* wire, uint64_t stride, uint64_t count, uint64_t tag_off,
                      uint64_t aad_off, uint32_t nrec, uint8_t* cache_k, uint8_t* cache_v,
                      uint64_t slot_bytes, const int64_t* slots, const uint32_t* kinds,
                      uint32_t bits, uint32_t heads, uint32_t dim, uint32_t layer,
                      uint32_t* status, uint32_t threads)
{
    if (threads == 0) threads = 1;
    if (threads > nrec) threads = nrec ? nrec : 1;
    pthread_t* tid = (pthread_t*)calloc(threads, sizeof(pthread_t));
    layer_job* jobs = (layer_job*)calloc(threads, sizeof(layer_job));
    uint8_t* scratch = NULL;
    if (bits) scratch = (uint8_t*)malloc((size_t)threads * (count + 64));
    struct timespec a, b;
    clock_gettime(CLOCK_MONOTONIC, &a);
    for (uint32_t t = 0; t < threads; ++t) {
        layer_job* j = &jobs[t];
        j->direction = direction;
        j->key = key; j->iv12 = iv12; j->wire = wire;
        j->stride = stride; j->count = count; j->tag_off = tag_off; j->aad_off = aad_off;
        j->nrec = nrec;
        j->cache[0] = cache_k; j->cache[1] = cache_v;
        j->slot_bytes = slot_bytes; j->slots = slots; j->kinds = kinds;
        j->bits = bits; j->heads = heads; j->dim = dim; j->layer = layer;
        j->scratch = scratch ? scratch + (uint64_t)t * (count + 64) : NULL;
        j->status = status;
        j->r0 = (uint32_t)((uint64_t)nrec * t / threads);
        j->r1 = (uint32_t)((uint64_t)nrec * (t + 1) / threads);
        if (threads == 1) layer_worker(j);
        else pthread_create(&tid[t], NULL, layer_worker, j);
    }
    if (threads > 1)
        for (uint32_t t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    clock_gettime(CLOCK_MONOTONIC, &b);
    free(scratch);
    free(jobs);
    free(tid);
    return (int64_t)(b.tv_sec - a.tv_sec) * 1000000000LL + (b.tv_nsec - a.tv_nsec);
}

/*
 * X25519 and keyed BLAKE2b through OpenSSL (EVP_PKEY_X25519, EVP_MAC
 * "BLAKE2BMAC"): an implementation independent of the restatement in
 * oracle/agreement.py and of the device code, for the session key agreement
 * (secure_infer.cpp:447-521, key_agreement.aicpu:9-49).
 */
#include <openssl/core_names.h>
#include <openssl/params.h>

int si_ossl_x25519(const uint8_t scalar[32], const uint8_t u[32], uint8_t out[32])
{
    EVP_PKEY* priv = EVP_PKEY_new_raw_private_key(EVP_PKEY_X25519, NULL, scalar, 32);
    EVP_PKEY* peer = EVP_PKEY_new_raw_public_key(EVP_PKEY_X25519, NULL, u, 32);
    EVP_PKEY_CTX* ctx = priv ? EVP_PKEY_CTX_new(priv, NULL) : NULL;
    size_t len = 32;
    int rc = -1;
    if (ctx && peer && EVP_PKEY_derive_init(ctx) == 1 && EVP_PKEY_derive_set_peer(ctx, peer) == 1 &&
        EVP_PKEY_derive(ctx, out, &len) == 1 && len == 32)
        rc = 0;
    EVP_PKEY_CTX_free(ctx);
    EVP_PKEY_free(peer);
    EVP_PKEY_free(priv);
    return rc;
}

int si_ossl_x25519_public(const uint8_t scalar[32], uint8_t out[32])
{
    EVP_PKEY* priv = EVP_PKEY_new_raw_private_key(EVP_PKEY_X25519, NULL, scalar, 32);
    size_t len = 32;
    int rc = (priv && EVP_PKEY_get_raw_public_key(priv, out, &len) == 1 && len == 32) ? 0 : -1;
    EVP_PKEY_free(priv);
    return rc;
}

int si_ossl_blake2b_keyed(const uint8_t* key, size_t key_len, const uint8_t* msg, size_t msg_len, uint8_t* out,
                          size_t out_len)
{
    EVP_MAC* mac = EVP_MAC_fetch(NULL, "BLAKE2BMAC", NULL);
    EVP_MAC_CTX* ctx = mac ? EVP_MAC_CTX_new(mac) : NULL;
    OSSL_PARAM params[2];
    params[0] = OSSL_PARAM_construct_size_t(OSSL_MAC_PARAM_SIZE, &out_len);
    params[1] = OSSL_PARAM_construct_end();
    size_t len = 0;
    int rc = -1;
    if (ctx && EVP_MAC_init(ctx, key, key_len, params) == 1 && EVP_MAC_update(ctx, msg, msg_len) == 1 &&
        EVP_MAC_final(ctx, out, &len, out_len) == 1 && len == out_len)
        rc = 0;
    EVP_MAC_CTX_free(ctx);
    EVP_MAC_free(mac);
    return rc;
}
