// Host-visible launch interface of the HIP kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "secure_infer_gpu.h"

#include <hip/hip_ext.h>

namespace si {

struct GcmCtx;
struct RecAcc;

// A batch of records.  single != 0: one record with explicit pointers
// (src/dst/aad/tag/status/ks/iv).  Otherwise records r = 0..nrec-1 live in a
// wire buffer (stride wire_stride) and map to paged-cache slots.
struct RecBatch {
    int single;
    int encrypt;  // layer form: 1 = writeback (cache -> wire), 0 = reload
    // single-record form
    const uint8_t* src;
    uint8_t* dst;
    const uint8_t* aad;
    uint8_t* tag;
    uint32_t* status;
    const uint8_t* ks;
    uint32_t iv[4];  // single: full IV; layer: iv[0] = salt word, iv[3] = counter start
    // layer form
    const uint8_t* wire;
    uint64_t wire_stride;
    uint64_t tag_off, status_off, aad_off;
    uint8_t* cache[2];
    uint64_t slot_bytes;
    const int64_t* slots;
    int64_t nslots;        // slot ids outside [0, nslots) fail the record, nothing is touched
    uint32_t n_k;
    const uint32_t* ivs;   // 4 words per record, or null: derive from nonce_base + r
    uint64_t nonce_base;   // session_nonce + ticket of record 0
    uint8_t* staging;      // codec: plaintext packets go here instead of the cache
    uint64_t staging_stride;
    uint32_t* fail_count;
};

// Most workgroups whose shares the host lays out one by one (kernel
// argument space); larger launches split the rows equally.
#define SI_MAX_WG 768

// Work decomposition shared by all records of a batch (uniform sizes).
struct Sched {
    uint32_t nrec;       // records
    uint32_t rows;       // R: rows of T blocks per record, ceil((a + n) / T) (at least 1)
    uint32_t nwg;        // W workgroups: W >= nrec (a share spans at most R rows), or
                         // ceil(nrec / 2) with pairs (a share is two whole records)
    uint32_t use_starts; // 1: workgroup w owns rows [starts[w], starts[w+1]); 0: an equal split
    uint32_t starts[SI_MAX_WG + 1];  // share boundaries in the records' concatenated rows
    uint32_t a;          // AAD blocks
    uint32_t n;          // payload blocks
    uint32_t aad_bytes;
    uint64_t bytes;      // payload bytes
    uint32_t lh[4];      // L * H, L = [len(A)]_64 || [len(C)]_64: the length block's GHASH term
    uint32_t ek_row0;    // 1: row 0 holds AAD block a-1 and a ciphertext block, and the tag
                         // mask E_K(J0) rides on row 0's keystream pass
    uint32_t pairs;      // 1: workgroup w owns the whole records 2w and 2w+1
    uint4* park;         // pairs: each thread's segment-0 product during segment 1
                         // (one uint4 per thread of each workgroup)
    uint32_t* status_out;  // layer form, optional: record r's status also at
                           // status_out[r] (one contiguous array, device or
                           // mapped pinned host memory)
    const uint32_t* gate;  // optional: when *gate == 0 every workgroup returns
                           // at once (an allocation-free call that does not own
                           // the GPU's scratch; see noalloc_finish)
    uint64_t* clock;       // optional: clock stamps of a measured launch (ClockProbe)
};
// Scratch of the allocation-free reload (secure_infer_gpu_reload_layer_noalloc):
// one device array per GPU, [control words][accumulators of up to
// SI_NOALLOC_MAX_RECORDS records][parking area of pairs][codec staging].
// Control word 0 is the owner token (0 = free), word 1 the token sequence.
#define SI_NOALLOC_SCRATCH_BYTES (64ull << 20)
#define SI_NOALLOC_MAX_RECORDS 8192u
#define SI_NOALLOC_CTRL_BYTES 256u
#define SI_NOALLOC_ACC_BYTES (uint64_t(SI_NOALLOC_MAX_RECORDS) * 32u)
// Token the test hook holds the scratch with (never handed to a call).
#define SI_NOALLOC_TEST_TOKEN 0xffffffffu
// Device address of the current GPU's scratch; on a device's first call its
// control words and accumulators are zeroed on `stream` and waited for
// (a capturing stream skips this: the array is zero when the module loads).
// nullptr on failure.
uint8_t* noalloc_scratch(hipStream_t stream);

// Exclusive use of the scratch by one allocation-free call, without any
// wait on the device (a wave that spun for another stream's release could
// hold a hardware queue the release is queued behind):
//   acquire: one thread draws a token (never 0 or the test token) and
//            compare-and-swaps the owner word from 0 to it; `cell` (4 bytes
//            of the call's own memory) receives the token, or 0 when the
//            scratch is held by another call;
//   the call's kernels run with gate = cell and return at once on 0;
//   finish:  owner -> 0 if the call held it; a call that did not hold it
//            fails every record closed instead: its output extent zeroed
//            (bf16 payload, or the whole bf16 block of a codec record),
//            status 0 in the wire record and status_out, fail_count += nrec.
struct NoallocFinish {
    uint32_t* ctrl;
    const uint32_t* cell;
    uint8_t* wire;
    uint64_t wire_stride, status_off;
    uint8_t* cache[2];
    uint64_t slot_bytes, out_bytes;
    const int64_t* slots;
    int64_t nslots;
    uint32_t nrec, n_k;
    uint32_t* status_out;
    uint32_t* fail_count;
};
hipError_t launch_noalloc_acquire(hipStream_t stream, uint32_t* ctrl, uint32_t* cell);
hipError_t launch_noalloc_finish(hipStream_t stream, const NoallocFinish& f);
// Test hook: hold (1) or release (0) the scratch with SI_NOALLOC_TEST_TOKEN.
hipError_t launch_noalloc_test_hold(hipStream_t stream, uint32_t* ctrl, int hold);

// Clock stamps of a measured layer: lane 0 of every wave of the layer's
// kernels writes the device's constant-rate clock (wall_clock64) when the
// wave starts and when it ends, two words per wave (wave w of a kernel:
// words 2w, 2w + 1 of that kernel's share), the kernels' shares one after
// another from `stamps`.  The layer's kernel time is the last end minus the
// first start.  A kernel whose share does not fit in `words` stamps nothing
// and sets `overflow`.
struct ClockProbe {
    uint64_t* stamps = nullptr;  // device memory
    uint64_t words = 0;
    uint64_t used = 0;
    bool overflow = false;

    uint64_t* take(uint64_t waves)
    {
        if (!stamps || used + 2 * waves > words) {
            overflow = overflow || stamps != nullptr;
            return nullptr;
        }
        uint64_t* p = stamps + used;
        used += 2 * waves;
        return p;
    }
};

// Events a timed launch records at its kernel's dispatch start and end
// (hipExtLaunchKernel: the interval a kernel trace reports, without the
// launch gaps an event recorded between kernels adds), and the clock probe
// of a measured launch.  Null: a plain launch.
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    ClockProbe* clock = nullptr;
};

hipError_t launch_gcm(int mode, hipStream_t stream, const GcmCtx* ctx, const RecBatch& b,
                      const Sched& s, RecAcc* acc, bool aligned, const LaunchEvents& ev = LaunchEvents());
// Verify-before-release, second launch (after a MODE_VERIFY launch over the
// same batch wrote every status): each record's plaintext to its
// destination if its status is 1, zeros otherwise.  nrec records of `bytes`.
#define SI_RELEASE_THREADS 512
// cus: the device's compute units (the grid's size).
hipError_t launch_release(hipStream_t stream, const GcmCtx* ctx, const RecBatch& b, uint32_t nrec, uint64_t bytes,
                          bool aligned, const uint32_t* gate, uint32_t cus,
                          const LaunchEvents& ev = LaunchEvents());
hipError_t launch_ctr(hipStream_t stream, const GcmCtx* ctx, const uint8_t* in, uint8_t* out,
                      uint64_t bytes, const uint32_t iv[4]);
hipError_t launch_auth_gate(hipStream_t stream, uint8_t* data, const uint32_t* status,
                            uint64_t bytes);

// One GHASH (the reference's secure_infer_ghash task, ghash.aicpu:978-1045):
// output = GHASH_H(aad || input || lengths) (^ tag_mask with FINALIZE_TAG);
// with VERIFY_TAG the status is 1 iff output equals expected_tag (else 1);
// with XOR_ON_SUCCESS plaintext = (input ^ keystream) & (0 - status),
// written after the verdict.  Any pointer may be unaligned.
// (flags: SI_GHASH_* of secure_infer_gpu.h)
struct GhashJob {
    const uint8_t* input;
    const uint8_t* aad;
    const uint8_t* tag_mask;
    const uint8_t* expected_tag;
    const uint8_t* keystream;
    uint8_t* plaintext;
    uint32_t* status;  // may be null
    uint8_t* output;   // 16 bytes
    uint64_t input_bytes, aad_bytes;
    uint32_t flags;
};
// ctx: a context of H (the powers H^0 .. H^(SI_T + 1) and the tables of H^SI_T).
hipError_t launch_ghash(hipStream_t stream, const GcmCtx* ctx, const GhashJob& j);

// Codec kernels (si_codec.hip).
struct CodecBatch {
    uint32_t nrec, n_k, bits, heads, dim, layer;
    uint8_t* cache[2];
    uint64_t slot_bytes;
    const int64_t* slots;
    int64_t nslots;
    uint8_t* staging;       // packets, one per record
    uint64_t staging_stride;
    uint64_t qbytes, sbytes, width;
    const uint32_t* gate;   // as Sched::gate (dequantiser only)
    uint64_t* clock;        // as Sched::clock
};
hipError_t launch_dequant_scatter(hipStream_t stream, const CodecBatch& b, const LaunchEvents& ev = LaunchEvents());
hipError_t launch_gather_quant(hipStream_t stream, const CodecBatch& b, const LaunchEvents& ev = LaunchEvents());

// Session key agreement and device-side context set-up (si_agree.hip).
struct AgreeIo {
    uint8_t host_public[32];    // in
    uint8_t challenge[32];      // in
    uint8_t device_public[32];  // out
    uint8_t proof[32];          // out: BLAKE2b-32 keyed by the key over the challenge
    int32_t status;             // out: 0 done; 1, 2 or 3 failed (the step it stopped at)
    uint32_t pad[7];
};
// Host seed mixed with the device's clock jitter (a kernel argument).
struct AgreeSeed {
    uint8_t b[32];
};
// Entropy pool (`pool`: SI_AGREE_POOL_WORDS u32, `counter`: one u32) and the
// agreement; the 16-byte key is written to `key_out` (device memory only).
// Every pointer is device memory.
#define SI_AGREE_POOL_WORDS (512u * 256u)
hipError_t launch_agree(hipStream_t stream, const uint8_t* host_public, const uint8_t* challenge,
                        const AgreeSeed& seed, uint32_t* pool, uint32_t* counter, uint8_t* key_out,
                        uint8_t* device_public, uint8_t* proof, int32_t* status);
// GcmCtx (+ npow powers) from a device-resident 16-byte key; te0 is public.
hipError_t launch_ctx_build(hipStream_t stream, const uint8_t* key, const uint32_t* te0, GcmCtx* ctx,
                            uint32_t npow);
hipError_t launch_zero_bytes(hipStream_t stream, uint8_t* p, uint32_t n);
hipError_t launch_x25519_test(hipStream_t stream, const uint8_t* scalar, const uint8_t* u, uint8_t* out);
hipError_t launch_blake2b_test(hipStream_t stream, const uint8_t* key, uint32_t key_len, const uint8_t* msg,
                               uint64_t msg_len, uint8_t* out, uint32_t out_len);

}  // namespace si
