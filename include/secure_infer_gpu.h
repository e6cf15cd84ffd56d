/*
 * secure_infer for MI355X (gfx950): C-ABI of libsecure_infer.so.
 *
 * The library implements the authenticated KV reload (H2D) and writeback
 * (D2H) data plane of secure_infer: AES-128-GCM records (one per 128-token
 * block, layer and K/V kind) verified and decrypted (or encrypted and tagged)
 * on the GPU by hand-written HIP kernels, with the int8/int4 transport codec
 * and the paged-cache scatter/gather in the same launch sequence.
 *
 * Conventions (same as the reference's device ABI, launcher.asc:23-524):
 *   - every function returns 0 when the work was enqueued and -1 on a null or
 *     zero argument or a launch failure;
 *   - all buffer pointers are device addresses unless stated otherwise;
 *   - work is asynchronous on `stream`; authentication failure is data:
 *     the record's status word is 0 and its output is all zeros, success
 *     writes status 1 (ghash.aicpu:637-648, 1051-1068).
 *
 * A "record" on the wire is [ciphertext count B][zero pad to 32][tag 16]
 * [status 16][AAD 64], the reference's H2D wire record
 * (secure_infer.cpp:6319-6320, 6379-6388, 6529-6537, 6654-6657).
 */
#ifndef SECURE_INFER_GPU_H
#define SECURE_INFER_GPU_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* 1. Kernel-level entry points.  Same argument order and meaning as the
 *    reference's secure_infer_aicpu_*_do launchers (launcher.asc), with a
 *    hipStream_t in place of the ACL stream.  `key` (16 B) and `hash_subkey`
 *    (H = E_K(0^128), 16 B) are device buffers; the library reads them back
 *    once per call to select its per-key tables, so these calls wait for
 *    work already queued on `stream`.                                     */

/* launcher.asc:214-241, ghash.aicpu:594-651 */
int secure_infer_gpu_gcm_decrypt_verify_do(
    hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
    void* expected_tag, void* plaintext_output, void* status_output,
    uint64_t bytes, uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2,
    uint32_t iv_word3);

/* launcher.asc:245-275 */
int secure_infer_gpu_gcm_decrypt_verify_aad_do(
    hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
    void* expected_tag, void* plaintext_output, void* status_output,
    uint64_t bytes, uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2,
    uint32_t iv_word3, void* aad, uint64_t aad_bytes);

/* launcher.asc:279-308, ghash.aicpu:656-699 */
int secure_infer_gpu_gcm_encrypt_tag_do(
    hipStream_t stream, void* plaintext, void* key, void* hash_subkey,
    void* ciphertext_output, void* tag_output, uint64_t bytes,
    uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2, uint32_t iv_word3,
    void* aad, uint64_t aad_bytes);

/* launcher.asc:407-435, ghash.aicpu:780-827 */
int secure_infer_gpu_gcm_verify_only_aad_do(
    hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
    void* expected_tag, void* status_output, uint64_t bytes,
    uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2, uint32_t iv_word3,
    void* aad, uint64_t aad_bytes);

/* launcher.asc:343-376, ghash.aicpu:705-773 */
int secure_infer_gpu_gcm_verify_xor_aad_do(
    hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
    void* expected_tag, void* keystream, void* plaintext_output,
    void* status_output, uint64_t bytes, uint32_t iv_word0, uint32_t iv_word1,
    uint32_t iv_word2, uint32_t iv_word3, void* aad, uint64_t aad_bytes);

/* launcher.asc:134-155, ghash.aicpu:517-535 */
int secure_infer_gpu_aes_ctr_do(
    hipStream_t stream, void* input, void* key, void* output, uint64_t bytes,
    uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2, uint32_t iv_word3);

/* launcher.asc:160-179, ghash.aicpu:537-554 */
int secure_infer_gpu_keystream_do(
    hipStream_t stream, void* key, void* output, uint64_t bytes,
    uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2, uint32_t iv_word3);

/* launcher.asc:116-132, ghash.aicpu:1051-1068: zero `bytes` of `data`
 * unless *status == 1. */
int secure_infer_gpu_auth_gate_do(hipStream_t stream, void* data, void* status,
                                  uint64_t bytes);

/* launcher.asc:312-341 / 378-405: the AAD-less forms of the two above. */
int secure_infer_gpu_gcm_verify_xor_do(
    hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
    void* expected_tag, void* keystream, void* plaintext_output,
    void* status_output, uint64_t bytes, uint32_t iv_word0, uint32_t iv_word1,
    uint32_t iv_word2, uint32_t iv_word3);
int secure_infer_gpu_gcm_verify_only_do(
    hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
    void* expected_tag, void* status_output, uint64_t bytes,
    uint32_t iv_word0, uint32_t iv_word1, uint32_t iv_word2, uint32_t iv_word3);

/* launcher.asc:440-486, ghash.aicpu:834-940: up to 4 records of one key and
 * size, each verified and released as by secure_infer_gpu_gcm_verify_xor_aad_do.
 * The pointer arrays are host arrays of device pointers; iv_words holds 4
 * words per record; aads may be NULL when aad_bytes is 0. */
#define SI_GCM_VERIFY_XOR_BATCH_MAX 4u
int secure_infer_gpu_gcm_verify_xor_batch_do(
    hipStream_t stream, void* key, void* hash_subkey, void* const* ciphertexts,
    void* const* expected_tags, void* const* keystreams,
    void* const* plaintext_outputs, void* const* status_outputs,
    void* const* aads, uint64_t bytes, uint64_t aad_bytes,
    const uint32_t* iv_words, uint32_t count);

/* launcher.asc:184-210, ghash.aicpu:559-580: up to 32 CTR keystreams of
 * one key and length (outputs: host array of device pointers). */
#define SI_AES_KEYSTREAM_BATCH_MAX 32u
int secure_infer_gpu_keystream_batch_do(
    hipStream_t stream, void* key, void* const* outputs,
    const uint32_t* iv_words, uint64_t bytes, uint32_t count);

/* launcher.asc:75-114, ghash.aicpu:978-1045: output (16 B) = GHASH_H over
 * aad || input || [bits(aad)]_64 || [bits(input)]_64, XORed with tag_mask
 * under SI_GHASH_FINALIZE_TAG; under SI_GHASH_VERIFY_TAG the status is 1
 * iff output equals expected_tag (1 without the flag); under
 * SI_GHASH_XOR_ON_SUCCESS plaintext_output = (input ^ keystream) masked to
 * zero on failure, written after the verdict.  status_output may be NULL.
 * Needs H only (no key). */
#define SI_GHASH_FINALIZE_TAG 1u
#define SI_GHASH_VERIFY_TAG 2u
#define SI_GHASH_XOR_ON_SUCCESS 4u
int secure_infer_gpu_ghash_do(
    hipStream_t stream, void* input, void* hash_subkey, void* output,
    void* aad, void* tag_mask, void* expected_tag, void* keystream,
    void* plaintext_output, void* status_output, uint64_t input_bytes,
    uint64_t aad_bytes, uint32_t flags);

/* launcher.asc:19-32, key_agreement.aicpu:9-49: the device half of the
 * session agreement (every pointer device memory: host_public 32 B and
 * challenge 32 B in; device_key 16 B, device_public 32 B, proof 32 B and an
 * int32 status out).  status: 0 done; 1, 2 or 3 the step it stopped at
 * (2: the shared secret is zero).  The device secret comes from clock
 * jitter on the GPU and a host seed, not from /dev/urandom.  The key stays
 * in device memory unless the caller copies it. */
int secure_infer_gpu_key_agreement_do(
    hipStream_t stream, void* host_public, void* challenge, void* device_key,
    void* device_public, void* proof, void* status);

/* ------------------------------------------------------------------ */
/* 2. Sessions and layer-level fused entry points.
 *
 * A session holds one AES-128 key on the device together with its GHASH
 * tables (the reference keeps the key device-resident per session,
 * secure_infer.cpp:449-609).  The IV of record r is
 *   iv_salt[4] || BE64(session_nonce + ticket) || BE32(2)
 * (secure_infer_derive_transfer_iv, secure_infer.cpp:274-300).            */

typedef struct si_session si_session;

/* Largest record (ciphertext / packet bytes) a session accepts: the kernels
 * address a record's payload with 32-bit byte offsets.  No reference
 * counterpart (its records are single KV blocks of at most a few MiB). */
#define SI_MAX_RECORD_BYTES 0x7fff0000ull

/* max_record_bytes: 1 .. SI_MAX_RECORD_BYTES, else -1. */
int secure_infer_gpu_session_create(const uint8_t key[16], const uint8_t iv_salt[4],
                                    uint64_t session_nonce, uint64_t max_record_bytes,
                                    si_session** out);
/* Destroy waits for the device, issues the calling thread's pending swaps,
 * drops the session's unconsumed prefetches, and leaves its observed swaps
 * without retry (a record that failed then fails its layer's wait).  No
 * other thread may still use the session. */
int secure_infer_gpu_session_destroy(si_session* session);
/* The reference's device session (secure_infer_experimental_device_session,
 * secure_infer.cpp:447-521; device half key_agreement.aicpu:9-49): an X25519
 * exchange between the host (OpenSSL) and a device kernel agrees on the
 * AES-128 key, key = BLAKE2b-16 keyed by the shared secret over
 * "SecureInfer X25519 BLAKE2b test v1" || host public || device public ||
 * challenge; the device proves it with BLAKE2b-32 keyed by the key over the
 * challenge; the IV salt is BLAKE2b-4 keyed by the shared secret over
 * "SecureInfer IV salt v1".  Only public values, the challenge, a host seed
 * and the proof cross PCIe: the device derives its X25519 secret from the
 * clock jitter of racing waves mixed with the seed (HIP exposes no device
 * random source), keeps the key in device memory and builds the kernels'
 * context (round keys, H, GHASH tables) there.  The host keeps its own copy
 * for OpenSSL sealing and verification.  0, or -1 (nothing created). */
int secure_infer_gpu_session_agree(uint64_t session_nonce, uint64_t max_record_bytes, si_session** out);
/* H = E_K(0^128) of the session (host copy, 16 B). */
int secure_infer_gpu_session_hash_subkey(const si_session* session, uint8_t out[16]);

/* Codec modes of the KV transport codec (transport_codec.py:9-19). */
enum {
    SI_CODEC_NONE = 0, /* bf16 records, ciphertext = raw KV block */
    SI_CODEC_INT8 = 8,
    SI_CODEC_INT4 = 4,
};

/* One layer of authenticated reload: records [0, n_k) are K blocks and
 * [n_k, nrec) are V blocks; record r decrypts into
 * cache[kind] + slots[r] * slot_bytes.  Replaces the per-layer swap_blocks
 * calls of NativeTransfer.single_layer_kv_transfer (native_layerwise.py:94-130)
 * and the staged decode_into of PipelinedTransfer (pipelined_codec.py:113-139). */
typedef struct si_reload_desc {
    const void* wire;         /* device: nrec records of wire_stride bytes      */
    uint64_t wire_stride;     /* >= align32(bytes) + 96                        */
    uint64_t bytes;           /* ciphertext bytes per record (count)           */
    uint32_t nrec;
    uint32_t n_k;
    const uint32_t* iv_words; /* device, 4 BE words per record; NULL: derive   */
    uint64_t ticket_base;     /* ticket of record 0 when iv_words == NULL      */
    void* cache_k;            /* device paged cache of this layer, kind 0      */
    void* cache_v;            /* device paged cache of this layer, kind 1      */
    uint64_t slot_bytes;      /* bytes of one 128-token block in the cache     */
    uint64_t nslots;          /* slots per cache; out-of-range ids fail closed */
    const int64_t* slots;     /* device, one slot id per record                */
    uint32_t codec_bits;      /* SI_CODEC_NONE / INT8 / INT4                   */
    uint32_t heads;           /* kv heads (codec only)                         */
    uint32_t head_dim;        /* head dim (codec only)                         */
    uint32_t layer;           /* layer index (codec header, status)            */
    void* staging;            /* device scratch, nrec*align32(bytes) (codec)   */
    uint32_t* fail_count;     /* device u32: += number of failed records; NULL ok */
    uint32_t* status_out;     /* optional: nrec u32, record r's status (1 / 0)
                                 also at status_out[r]; device memory or
                                 mapped pinned host memory; NULL ok          */
    uint32_t flags;           /* SI_RELOAD_* below; 0 = the fused default       */
} si_reload_desc;

/* si_reload_desc.flags.  SI_RELOAD_VERIFY_BEFORE_RELEASE: the reference's
 * order (ghash.aicpu:623-648, direct verified release secure_infer.cpp:
 * 5522-5538) -- a first launch computes every record's tag and status and
 * writes nothing else; a second decrypts each record into its slot (or the
 * codec staging) only if its status is 1 and writes zeros otherwise.  No
 * unverified byte ever reaches the cache, at the price of reading the
 * ciphertext twice.  The default (0) decrypts and hashes in one pass and
 * zeroes a failed record's slot before the launch sequence ends. */
enum { SI_RELOAD_VERIFY_BEFORE_RELEASE = 1u };

int secure_infer_gpu_reload_layer(hipStream_t stream, si_session* session,
                                  const si_reload_desc* desc);

/* secure_infer_gpu_reload_layer without any device allocation.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The kernels are the same; their scratch (GHASH
 * accumulators, the parking area of two-record shares and, with a codec, the
 * packet staging) lives in one 64 MiB device array per GPU
 * (SI_NOALLOC_SCRATCH_BYTES below, held until the process ends) instead of
 * per-stream workspaces and the caller's staging buffer: desc->staging must
 * be NULL.  Limits: at most 8192 records, and 256 B of control words +
 * 256 KiB of accumulators + pair parking (12 KiB per workgroup when the
 * records outnumber the CUs) + nrec * align32(bytes) of staging (codec only)
 * within the 64 MiB; a larger request returns -1 with a message on stderr.
 * The first call on a GPU clears the control words and accumulators on
 * `stream` and waits for it (a capturing stream skips the clear: the array
 * is zero when the library loads).
 * Every call on one GPU shares that GPU's array, so each call first takes it
 * for itself with a one-thread device kernel (compare-and-swap of an owner
 * word with a fresh token; the token is written into bytes 4..7 of record
 * 0's status slot, which must therefore be writable) and returns it with a
 * last kernel.  A call whose work overlaps another's on the same GPU (other
 * streams, other threads) and finds the array taken does not wait: it
 * touches no scratch and fails closed -- every record gets status 0 (wire
 * record and status_out), its output extent is zeroed (bf16 payload, or the
 * whole bf16 block of a codec record; slots out of range are not touched)
 * and fail_count grows by nrec.  So overlapping calls never mix their
 * scratch, and no record keeps unverified plaintext without being counted
 * as failed.  Callers that need every call to verify serialise them. */
int secure_infer_gpu_reload_layer_noalloc(hipStream_t stream, si_session* session,
                                          const si_reload_desc* desc);

/* Kernel timing of the calling thread's next layer call (one shot; no
 * reference counterpart -- the reference's per-copy profile rows,
 * secure_infer.cpp:1826-1951, time its AICPU tasks): the next
 * secure_infer_gpu_reload_layer, _reload_layer_noalloc or _writeback_layer
 * launches its first kernel with `start` and its last kernel with `stop` as
 * hipExtLaunchKernel events, which take the kernels' own dispatch start and
 * end times (an event recorded between kernels also times the launch gap).
 * Either may be NULL; both must have been created by the caller.  0, or -1
 * if both are NULL. */
int secure_infer_gpu_time_next_layer(hipEvent_t start, hipEvent_t stop);

/* Kernel clock of the calling thread's next `layers` layer calls (no
 * reference counterpart, as above): lane 0 of every wave of the kernels of
 * each of the next `layers` secure_infer_gpu_reload_layer,
 * _reload_layer_noalloc or _writeback_layer calls writes the device's
 * constant-rate clock (wall_clock64; rate from
 * secure_infer_gpu_clock_rate_khz) when the wave starts and when it ends
 * into `stamps` (device memory): layer call l (in call order) takes words
 * [l * words_per_layer, (l + 1) * words_per_layer), two per wave (start,
 * end), its kernels one after another.  A layer's kernel time is the latest
 * end minus the earliest start of the words it wrote.  Unlike the events
 * above it adds nothing to the launches (a hipExtLaunchKernel event pair
 * lengthens each launch it times), and arming every layer at once leaves the
 * calls back to back.  Words a launch does not reach keep their contents;
 * arming again drops what was armed.  0, or -1 on NULL / 0 / overflow. */
int secure_infer_gpu_clock_next_layers(uint64_t* stamps, uint64_t words_per_layer, uint32_t layers);

/* Words each of the first `layers` clocked calls wrote, into words_used[l]
 * (may be NULL); -1 if fewer calls were clocked since the arming, or a
 * kernel of one of them did not fit in words_per_layer (that kernel wrote no
 * stamps). */
int secure_infer_gpu_clock_layers_used(uint64_t* words_used, uint32_t layers);

/* Rate of that clock on the current device, in kHz.  0, or -1. */
int secure_infer_gpu_clock_rate_khz(uint64_t* khz);

/* One layer of writeback: record r gathers cache[kind] + slots[r]*slot_bytes,
 * optionally quantises it with the transport codec, encrypts it and writes the
 * ciphertext and tag into its wire record (the AAD must already be there).
 * Replaces the D2H branch of the reference (secure_infer.cpp:8076-8562 with
 * gcm_encrypt_tag, ghash.aicpu:656-699) plus transport_codec.encode. */
typedef struct si_writeback_desc {
    void* wire;
    uint64_t wire_stride;
    uint64_t bytes;           /* plaintext (packet) bytes per record           */
    uint32_t nrec;
    uint32_t n_k;
    const uint32_t* iv_words;
    uint64_t ticket_base;
    const void* cache_k;
    const void* cache_v;
    uint64_t slot_bytes;
    uint64_t nslots;
    const int64_t* slots;
    uint32_t codec_bits;
    uint32_t heads;
    uint32_t head_dim;
    uint32_t layer;
    void* staging;            /* device scratch, nrec*align32(bytes) (codec)   */
    uint32_t* fail_count;     /* device u32: += records with a bad slot id     */
} si_writeback_desc;

int secure_infer_gpu_writeback_layer(hipStream_t stream, si_session* session,
                                     const si_writeback_desc* desc);

/* Size helpers of the codec packet (transport_codec.py:22-42). */
uint64_t secure_infer_codec_width(uint32_t bits, uint32_t heads, uint32_t head_dim);
uint64_t secure_infer_wire_stride(uint64_t bytes);

/* ------------------------------------------------------------------ */
/* 3. Control plane with the reference's names and semantics.            */

/* secure_infer.cpp:261-272: process-monotonic ticket from 1. */
uint64_t secure_infer_new_transfer_ticket(void);
/* secure_infer.cpp:274-300 (GCM counter base 2). Returns 0, or -1 on ticket 0. */
int secure_infer_derive_transfer_iv(const uint8_t base_iv[16], uint64_t session_nonce,
                                    uint64_t ticket, uint64_t block_offset,
                                    uint8_t out_iv[16]);
/* secure_infer.cpp:1066-1091 (host address ranges -> layer / kind / block);
 * registering an existing [base, base + bytes) again re-labels it. */
void secure_infer_register_host_range_ex(const void* base, size_t bytes, uint32_t layer_id,
                                         uint32_t tensor_kind, size_t block_bytes);
/* secure_infer.cpp:1093-1097: layer and kind unknown (0xffffffff), no block size. */
void secure_infer_register_host_range(const void* base, size_t bytes);
void secure_infer_clear_host_ranges(void);
/* secure_infer.cpp:730-775: 64-B AAD for a registered host address.
 * Returns 1 on success, 0 on invalid arguments. */
int secure_infer_build_gcm_aad(const void* host_ptr, size_t bytes, uint8_t direction,
                               uint64_t transfer_ticket, uint64_t transfer_offset,
                               uint64_t session_nonce, uint8_t out[64]);
/* secure_infer.cpp:777-789: 1 if the ticket was not seen before, else 0.
 * The host transfer runtime reserves every ticket it seals under (H2D
 * :6439-6445, D2H :8096-8115) and refuses a swap whose tickets were used. */
int secure_infer_gcm_replay_reserve(uint64_t transfer_ticket);

/* secure_infer.cpp:1102-1148: drop every record sealed ahead of demand
 * (secure_infer_h2d_prefetch) that no swap has consumed; their tickets stay
 * used.  Call it when host blocks change after a prefetch.  EncodedStore
 * binds the first unconditionally (transport_codec.py:50); both do the same
 * here (this library has no address predictor to reset). */
void secure_infer_retire_transfer_prefetches(void);
void secure_infer_invalidate_transfer_prefetches(void);
/* No reference counterpart (a layer-wide form of secure_infer_h2d_prefetch_group
 * for callers that bracket a whole layer in one layer group): seals the K and
 * V swaps of `ngroups` causal groups of one layer -- group g is rows
 * [group_start[g], group_start[g] + group_rows[g]) of `mapping`, taken in
 * the order given -- into one pinned buffer laid out as the device layout of
 * a launch of exactly those swaps: [every group's K records][every group's V
 * records][IV words][slot ids].  Tickets follow the swaps' order (group 0's
 * K, its V, group 1's K, ...), the order the reference's grouped loading
 * assigns them (native_layerwise.py:96-129), so the records are the ones the
 * swaps would seal on demand.  The swaps, issued inside one layer group in
 * that order, then go to the device as one DMA and one launch.  0, or -1
 * (bad argument, an id outside the host pool, or the prefetch budget
 * SECURE_INFER_PREFETCH_MB spent: the swaps then seal on demand). */
int secure_infer_h2d_prefetch_layer(si_session* session, const void* k_base, const void* v_base,
                                    uint64_t host_block_bytes, uint64_t host_nblocks, const int64_t* mapping,
                                    const uint32_t* group_start, const uint32_t* group_rows, uint32_t ngroups,
                                    uint32_t layer, uint32_t codec_bits, uint32_t heads, uint32_t head_dim);
/* secure_infer.cpp:817-830: swaps served from prefetched records that were
 * ready / that had to wait for their sealing to finish / swaps sealed on
 * demand (the reference's ready / busy_fallback / missing_fallback; a busy
 * prefetch is waited for here, not abandoned). */
void secure_infer_get_transfer_prefetch_stats(uint64_t* ready, uint64_t* busy_fallback,
                                              uint64_t* missing_fallback);
/* secure_infer.cpp:5052-5070: records sealed ahead of demand and not yet consumed. */
uint64_t secure_infer_count_ready_unconsumed_gcm_tickets(void);

/* secure_infer.cpp:5883-5903: layer-group brackets (thread-local; they nest,
 * and only the outermost end issues; an end without a begin returns -1).
 * `expected` (of the outermost begin) is the group's record count.  Swaps of the group accumulate and go out as
 * few launches as their stream, layer and geometry allow (K swaps, then V
 * swaps, of one stream form one launch; at most SECURE_INFER_H2D_BATCH_MB of
 * records, default 64), issued at the latest by group_end, as the reference
 * batches a group's swaps (:5862-5881).  group_end returns -1 if issuing
 * them failed. */
int secure_infer_h2d_layer_group_begin(size_t expected);
int secure_infer_h2d_layer_group_end(void);

/* secure_infer.cpp:7303-7333: 0 if every record submitted for `layer` since
 * the last wait authenticated, -1 otherwise.  Waits for the layer's work.
 * Records sealed by secure_infer_h2d_swap inside a layer group are observed
 * one by one (the kernel stores each status into mapped pinned memory); a
 * record that failed is re-sealed once from its trusted host block under a
 * fresh ticket and reloaded on its stream, and the layer fails only if that
 * second attempt fails too (strict retry, :7316-7330).  Device-resident
 * records registered with secure_infer_recovery_track_layer have no host
 * copy: any failure among them is -1. */
int secure_infer_recovery_wait_layer_authentication(uint32_t layer);
/* secure_infer.cpp:5311-5314, 7336-7372: records observed after set_job_id
 * belong to that job; wait_job_authentication waits for every record of the
 * job on every layer (no retry) and returns 1 if all authenticated, 0 if any
 * failed and -1 if the job has no observed records. */
void secure_infer_recovery_set_job_id(uint64_t job_id);
int secure_infer_recovery_wait_job_authentication(uint64_t job_id);
/* Registers a reload of `layer` whose per-record statuses land in the device
 * u32 `fail_count` once `event` completes (library-internal bookkeeping used
 * by the Python layer driver). */
int secure_infer_recovery_track_layer(uint32_t layer, hipEvent_t event,
                                      const uint32_t* fail_count);

/* ------------------------------------------------------------------ */
/* 4. Host transfer runtime: host AES-GCM, pinned ring, copy streams.     */
/*                                                                        */
/* The reference turns every intercepted aclrtMemcpyAsync of a registered */
/* host range into one record (secure_infer.cpp:7729-8571).  ROCm has     */
/* nothing to interpose, so the maintainer replaces each swap_blocks call */
/* site with the explicit calls below; `mapping` is the swap_blocks       */
/* mapping, n int64 pairs (source block, destination block) in host       */
/* memory.  Host blocks are `host_block_bytes` apart from `host_base`:    */
/* bf16 KV blocks [128, heads, head_dim], or codec packets (rows of a     */
/* packet array, at least secure_infer_codec_width bytes).  AADs are      */
/* built from the registered host ranges (secure_infer_build_gcm_aad).    */
/* Like swap_blocks, which sees both tensors' shapes, the calls know the  */
/* pool sizes: a mapping entry outside [0, host_nblocks) or [0, nslots)   */
/* refuses the whole call (-1) before any work is queued.                 */

/* H2D reload of n blocks of one (layer, kind): host OpenSSL AES-128-GCM on
 * the library's worker pool into a pinned ring slot (inline_h2d_encrypt_commit,
 * secure_infer.cpp:6486-6550; slot ring :5174-5229, :5905-6059), DMA on the
 * ring's copy stream, then the fused verify + decrypt (+ dequantise) + paged
 * scatter on `stream` once the copy has landed.  Returns when the work is
 * queued; a ring slot is reused only after its kernel completed.  Rings,
 * copy streams and locks are per (device, stream), as the reference keeps
 * them per stream (:5389-5399).  Inside secure_infer_h2d_layer_group_begin/end
 * the records are sealed (or taken from a prefetch) by the call, but their
 * copy and kernel are issued with the group's other swaps (see above), and
 * every record is observed for secure_infer_recovery_wait_layer_authentication.  mapping pairs are (host
 * block, device slot).  fail_count (device u32, may be NULL): += records
 * that failed in this launch. */
int secure_infer_h2d_swap(hipStream_t stream, si_session* session, const void* host_base,
                          uint64_t host_block_bytes, uint64_t host_nblocks, void* dev_cache,
                          uint64_t slot_bytes, uint64_t nslots, const int64_t* mapping, uint32_t n,
                          uint32_t kind, uint32_t layer, uint32_t codec_bits, uint32_t heads,
                          uint32_t head_dim, uint32_t* fail_count);

/* Test-only fault injection of the reference's trust-boundary tests
 * (PIPE_GCM_TAMPER_H2D / _LAYER / _TENSOR, secure_infer.cpp:6139-6250, and
 * PIPE_GCM_TAMPER_D2H, :2451-2467): the next `shots` H2D records sealed from
 * host block `host_block` of (layer, kind) -- -1 matches any -- get their
 * first ciphertext byte flipped after sealing and before the DMA; the next
 * `shots` D2H records get theirs flipped in host memory before host
 * authentication.  0 shots disarms.  Production code never calls them. */
int secure_infer_test_tamper_h2d(int32_t layer, int32_t kind, int64_t host_block, uint32_t shots);
int secure_infer_test_tamper_d2h(uint32_t shots);
/* Test-only checks of the session agreement's device code (no reference
 * counterpart): X25519 (RFC 7748) and keyed BLAKE2b (RFC 7693) run by one
 * device lane; the kernels' context built on the device (on_device = 1) or
 * on the host (0) from a key, written to out (cap bytes; out = NULL returns
 * the size).  Production code never calls them. */
/* Test-only fault injection for the next secure_infer_gpu_session_agree
 * (one shot; no reference counterpart): mode 1 flips a byte of the device's
 * proof as it reaches the host, mode 2 sends the all-zero (low-order) public
 * value to the device; either makes the agreement return -1.  0 disarms. */
int secure_infer_test_tamper_agree(uint32_t mode);
/* Test-only (no reference counterpart): holds (hold != 0) or releases the
 * current GPU's allocation-free scratch with a token no call receives, on
 * `stream`, so a test can make secure_infer_gpu_reload_layer_noalloc find it
 * taken.  0 or -1.  Production code never calls it. */
int secure_infer_test_noalloc_hold(hipStream_t stream, int hold);
/* Test-only (no reference counterpart): the calling thread's next
 * verify-before-release reload stops after its first n launches (1: the
 * verification alone, so a test can see that it writes nothing but
 * statuses); 0 disarms.  0 or -1.  Production code never calls it. */
int secure_infer_test_strict_phases(int n);
int secure_infer_test_x25519(const uint8_t scalar[32], const uint8_t u[32], uint8_t out[32]);
int secure_infer_test_blake2b(const uint8_t* key, uint32_t key_len, const uint8_t* msg, uint64_t msg_len,
                              uint8_t* out, uint32_t out_len);
int64_t secure_infer_test_context_image(const uint8_t key[16], uint64_t max_record_bytes, int on_device,
                                        void* out, uint64_t cap);

/* Ahead-of-demand sealing (the reference's CPU ciphertext prefetch pool,
 * secure_infer.cpp:3264-3710): queues the host seal of the swap with these
 * arguments on the worker pool and returns; tickets are reserved now, in
 * mapping order.  The next secure_infer_h2d_swap with the same session,
 * host pool, kind, layer, codec and host-block column of its mapping copies
 * the sealed records instead of sealing (waiting for them if still being
 * sealed).  The records snapshot the host blocks when sealed: call
 * secure_infer_retire_transfer_prefetches if the blocks change before the
 * swap.  Pinned memory for prefetches is bounded by SECURE_INFER_PREFETCH_MB
 * (default 2048); beyond it the call returns -1 and the swap seals on demand. */
int secure_infer_h2d_prefetch(si_session* session, const void* host_base, uint64_t host_block_bytes,
                              uint64_t host_nblocks, const int64_t* mapping, uint32_t n, uint32_t kind,
                              uint32_t layer, uint32_t codec_bits, uint32_t heads, uint32_t head_dim);
/* A layer group's two swaps at once (no reference counterpart; the same
 * prefetch for the K swap of `mapping` from k_base followed by the V swap of
 * the same mapping from v_base, tickets in that order).  The records of both
 * halves and the group's slot ids share one pinned buffer, so a launch of
 * exactly this group (its K swap then its V swap on one stream) goes to the
 * device in one copy. */
int secure_infer_h2d_prefetch_group(si_session* session, const void* k_base, const void* v_base,
                                    uint64_t host_block_bytes, uint64_t host_nblocks, const int64_t* mapping,
                                    uint32_t n, uint32_t layer, uint32_t codec_bits, uint32_t heads,
                                    uint32_t head_dim);

/* secure_infer.cpp:6085-6137: the H2D ledger.  With
 * SECURE_INFER_H2D_PROFILE=<path> every launch appends one CSV row (layer,
 * kind -- 0 K, 1 V, 2 both --, records, record_bytes, source, seal_us,
 * h2d_copy_us, kernel_us) once its work is complete; with
 * SECURE_INFER_H2D_PROFILE_RECORDS=1 as well, one row per record in the
 * reference's per-copy columns (secure_infer.cpp:1846-1847): the record's
 * own seal time and prefetch hit, its launch's enqueue times and device
 * phases.  Flush writes the rows of completed launches, drain waits for
 * every pending launch first. */
void secure_infer_flush_completed_h2d_profile(void);
void secure_infer_drain_h2d_profile_after_job(void);
/* No reference counterpart: pauses (1) or resumes (0) the ledger's rows and
 * their timing events, so a caller can time transfers without the ledger's
 * own cost and record a ledger over other ones. */
void secure_infer_pause_h2d_profile(int paused);

/* Threads of the host crypto pool (the calling thread included): the CPUs of
 * the process affinity mask, or SECURE_INFER_HOST_THREADS.  No reference
 * counterpart (its pools are sized by PIPE_D2H_CPU_WORKERS, :2568-2629). */
int secure_infer_host_threads(void);

/* D2H batch / group API (same names, thread-local contexts and returns as
 * secure_infer.cpp:2707-2970): batch_begin returns 1 (-1 when nested),
 * group_begin 1 (-1 without a batch or inside a group), group_end and
 * batch_device_barrier 0, batch_end 0 when every record of the batch
 * authenticated on the host and -1 otherwise (failed records are zeroed). */
int secure_infer_d2h_batch_begin(size_t expected_tasks);
int secure_infer_d2h_group_begin(size_t expected_tasks);
int secure_infer_d2h_group_end(void);
int secure_infer_d2h_batch_device_barrier(void);
int secure_infer_d2h_batch_end(void);

/* Inside an open D2H group: gather (+ quantise) and seal n device blocks of
 * one (layer, kind) on `stream` (the hook's D2H branch, secure_infer.cpp:
 * 8076-8562, with gcm_encrypt_tag, ghash.aicpu:656-699), copy the records to
 * pinned memory on the library's D2H stream, then the worker pool
 * authenticates and decrypts each into host_base + block*host_block_bytes
 * (d2h_host_decrypt_one, secure_infer.cpp:2470-2547).  mapping pairs are
 * (device slot, host block).  A batch's swaps of one stream and layer (K
 * before V, across groups; up to a quarter of the records the batch
 * announced, at least 8 MiB and at most SECURE_INFER_D2H_LAUNCH_MB = 64)
 * go out as one launch, issued by the next swap that does not fit
 * it or at the latest by batch_device_barrier / batch_end; a per-device
 * thread hands each launch to the pool once its copy is done.  At most 6
 * launches and SECURE_INFER_D2H_INFLIGHT_MB (128) of buffers are in flight
 * per device; an issue beyond that waits.  A failed record is zeroed in the
 * host pool and makes batch_end return -1 (the reference zeroes and aborts;
 * SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE=1 aborts too, after the zeroing).
 * Stream order of the source reads: the device reads a swap's slots when its
 * launch is issued, which can be as late as batch_device_barrier (the
 * reference enqueues each swap's read at the call).  So work the caller
 * queues on `stream` after a swap must not write that swap's source slots
 * until batch_device_barrier has returned; work queued after the barrier is
 * ordered behind every read of the batch.  The reference's own D2H driver
 * calls the barrier right after its last group (npu_predict.py:874-916). */
int secure_infer_d2h_swap(hipStream_t stream, si_session* session, const void* dev_cache,
                          uint64_t slot_bytes, uint64_t nslots, void* host_base,
                          uint64_t host_block_bytes, uint64_t host_nblocks, const int64_t* mapping,
                          uint32_t n, uint32_t kind, uint32_t layer, uint32_t codec_bits,
                          uint32_t heads, uint32_t head_dim);

/* Library build / device information. */
const char* secure_infer_gpu_version(void);
/* Tuning: minimum rows (of 256 blocks) of one workgroup's share of a layer's
 * rows, 1..256 (default 3); a launch spreads the rows of all records over one
 * workgroup per CU.  No reference counterpart; used by the benchmark sweep and
 * the tests (small values force shares that straddle records). */
int secure_infer_gpu_set_chunk_rows(int jmax);
/* Tuning: cost, in rows, charged to a workgroup share that straddles two
 * records when the launch lays out its shares, 0..256 (default 6); 0 lets
 * shares straddle wherever a record ends inside one.  No reference
 * counterpart; used by the tests to force straddling shares. */
int secure_infer_gpu_set_straddle_rows(int rows);
/* Inspection: the share layout a layer launch of nrec records of `bytes`
 * payload and `aad_bytes` AAD bytes would use on a device with `cus` compute
 * units (1..768) under the current tuning.  The host computes it alone; no
 * device call is made.  info_out[0..4]: workgroups W, rows R per record
 * (256 GHASH blocks each), 1 if the W shares are laid out one by one
 * (their boundaries in the records' concatenated rows go to starts_out[0..W],
 * which needs cap >= W + 1) or 0 for W equal shares, 1 if every workgroup
 * takes two whole records, 1 if a record's first row also holds ciphertext.
 * Returns 0, or -1 on invalid arguments.  No reference counterpart; used by
 * the tests to check the layout's invariants over many shapes. */
int secure_infer_gpu_layout(uint32_t nrec, uint64_t bytes, uint64_t aad_bytes, uint32_t cus,
                            uint32_t* info_out, uint32_t* starts_out, uint32_t cap);

#ifdef __cplusplus
}
#endif
#endif
