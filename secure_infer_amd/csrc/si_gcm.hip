// AES-128-GCM record kernels for gfx950.
//
// One launch processes a batch of records.  Each record's GHASH input is the
// block sequence X = AAD || C || L (SP 800-38D), m = a + n + 1 blocks, and
// GHASH = XOR_k X_k * H^(m-k).  X is cut into R rows of T blocks counted from
// its end (row R-1 ends with L; row 0 may start before X), and thread t of a
// workgroup owns block t of each of its rows, so every row is one coalesced
// 4 KiB sweep.  Each record's rows are split into K contiguous chunks, one
// per workgroup.  Per thread:
//   * CTR: keystream of counter iv3 + k for ciphertext block k (32-bit wrap,
//     ghash.aicpu:174-221), XORed into the data and stored;
//   * GHASH: Horner with H^T over the thread's blocks (LDS tables), then one
//     generic multiply by H^((R - q1)*T + T - t) from the per-key power table
//     (q1 = end row of the chunk), which places the
//     thread's partial at its true exponent.
// Partials are XOR-reduced over the workgroup and then across workgroups with
// device-scope atomics; a ticket names the workgroup that completes a
// record, which compares the tag in constant time, writes the
// status and, on failure, zeroes the record's output before the kernel ends.
// The zeroing must land after every plaintext store of the record:
// full-block stores are issued write-through (sc1, agent-coherent) and
// drained (s_waitcnt) before a workgroup takes its ticket; byte-granular
// stores (partial or unaligned blocks) fall back to an agent-scope release
// (L2 write-back) instead.
#include "si_device.h"
#include "si_kernels.h"

namespace si {

enum Mode : int {
    MODE_DECRYPT = 0,     // verify + decrypt, output zeroed on failure
    MODE_ENCRYPT = 1,     // encrypt + tag
    MODE_VERIFY = 2,      // tag check only
    MODE_VERIFY_XOR = 3,  // verify + XOR with a given keystream
};

template <bool kAligned>
__device__ __forceinline__ void load_block(const uint8_t* p, uint32_t valid, uint32_t w[4])
{
    if (kAligned && valid == 16u) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        return;
    }
    w[0] = w[1] = w[2] = w[3] = 0;
    for (uint32_t b = 0; b < valid; ++b) w[b >> 2] |= uint32_t(p[b]) << (8 * (b & 3));
}

template <bool kAligned>
__device__ __forceinline__ void store_block(uint8_t* p, uint32_t valid, const uint32_t w[4])
{
    if (kAligned && valid == 16u) {
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        return;
    }
    for (uint32_t b = 0; b < valid; ++b) p[b] = uint8_t(w[b >> 2] >> (8 * (b & 3)));
}

__device__ __forceinline__ void zero_bytes(uint8_t* p, uint64_t bytes, uint32_t tid,
                                           uint32_t nthreads)
{
    const bool aligned = (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
    if (aligned) {
        const uint64_t full = bytes >> 4;
        for (uint64_t i = tid; i < full; i += nthreads)
            reinterpret_cast<uint4*>(p)[i] = make_uint4(0, 0, 0, 0);
        for (uint64_t i = (full << 4) + tid; i < bytes; i += nthreads) p[i] = 0;
    } else {
        for (uint64_t i = tid; i < bytes; i += nthreads) p[i] = 0;
    }
}

struct RecView {
    const uint8_t* src;  // ciphertext (decrypt/verify) or plaintext (encrypt)
    uint8_t* dst;        // plaintext out (decrypt) or ciphertext out (encrypt)
    const uint8_t* aad;
    uint8_t* tag;        // expected tag, or tag output (encrypt)
    uint32_t* status;
    const uint8_t* ks;   // keystream (verify_xor)
    uint32_t iv[4];
    bool bad;            // block-table entry out of range: touch no cache memory
};

__device__ __forceinline__ RecView view_of(const RecBatch& b, uint32_t r)
{
    RecView v;
    if (b.single) {
        v.src = b.src;
        v.dst = b.dst;
        v.aad = b.aad;
        v.tag = b.tag;
        v.status = b.status;
        v.ks = b.ks;
        v.iv[0] = b.iv[0]; v.iv[1] = b.iv[1]; v.iv[2] = b.iv[2]; v.iv[3] = b.iv[3];
        v.bad = false;
        return v;
    }
    uint8_t* wire = const_cast<uint8_t*>(b.wire) + uint64_t(r) * b.wire_stride;
    const uint32_t kind = r < b.n_k ? 0u : 1u;
    const int64_t sid = b.slots[r];
    v.bad = sid < 0 || sid >= b.nslots;
    uint8_t* slot = b.cache[kind] + uint64_t(v.bad ? 0 : sid) * b.slot_bytes;
    uint8_t* stage = b.staging ? b.staging + uint64_t(r) * b.staging_stride : nullptr;
    uint8_t* plain = stage ? stage : slot;
    if (b.encrypt) {
        v.src = plain;
        v.dst = wire;
    } else {
        v.src = wire;
        v.dst = plain;
    }
    v.aad = wire + b.aad_off;
    v.tag = wire + b.tag_off;
    v.status = reinterpret_cast<uint32_t*>(wire + b.status_off);
    v.ks = nullptr;
    if (b.ivs) {
        const uint4 w = reinterpret_cast<const uint4*>(b.ivs)[r];
        v.iv[0] = w.x; v.iv[1] = w.y; v.iv[2] = w.z; v.iv[3] = w.w;
    } else {
        const uint64_t nonce = b.nonce_base + r;
        v.iv[0] = b.iv[0];
        v.iv[1] = uint32_t(nonce >> 32);
        v.iv[2] = uint32_t(nonce);
        v.iv[3] = b.iv[3];
    }
    return v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Write-through (sc1) 16-byte store: agent-coherent once s_waitcnt drains it,
// and measured faster than plain or non-temporal stores for this stream.
__device__ __forceinline__ void st_wt(__amdgpu_buffer_rsrc_t rsrc, uint64_t k, uint4 v)
{
    u32x4 w;
    w.x = v.x; w.y = v.y; w.z = v.z; w.w = v.w;
    __builtin_amdgcn_raw_buffer_store_b128(w, rsrc, uint32_t(k * 16u), 0, 16 /* sc1 */);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* p)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}

// One general row: any mix of AAD / ciphertext / length blocks, partial
// blocks and unaligned buffers.  Used for the few rows at a record's ends.
template <int kMode, bool kAligned, bool kWT>
__device__ __forceinline__ void row_general(const RecBatch& batch, const Sched& sch, const RecView& v,
                                            const uint32_t* aes, AesLane lane, const AesKeys& keys,
                                            uint32_t n0, uint32_t n1, uint32_t n2, int64_t i,
                                            uint32_t tail, uint32_t aad_tail, uint32_t y[4])
{
    if (i < 0) return;
    uint32_t x[4];
    if (i >= int64_t(sch.a) && i < int64_t(sch.a) + int64_t(sch.n)) {
        if (v.bad && !batch.staging) return;
        const uint64_t k = uint64_t(i - sch.a);
        const uint32_t valid = k == uint64_t(sch.n) - 1 ? tail : 16u;
        uint32_t in[4];
        load_block<kAligned>(v.src + 16 * k, valid, in);
        if (kMode == MODE_VERIFY) {
            x[0] = in[0]; x[1] = in[1]; x[2] = in[2]; x[3] = in[3];
        } else {
            uint32_t ks[4];
            if (kMode == MODE_VERIFY_XOR) {
                load_block<kAligned>(v.ks + 16 * k, valid, ks);
            } else {
                aes_ctr_block(aes, lane, keys, n0, n1, n2, v.iv[3] + uint32_t(k), ks);
            }
            uint32_t out[4] = {in[0] ^ ks[0], in[1] ^ ks[1], in[2] ^ ks[2], in[3] ^ ks[3]};
            if (kWT)  // every payload block is a full aligned block
                st_wt(rsrc_of(v.dst), k, make_uint4(out[0], out[1], out[2], out[3]));
            else
                store_block<kAligned>(v.dst + 16 * k, valid, out);
            if (kMode == MODE_ENCRYPT) {
                if (valid != 16u) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const int lo = 4 * w;
                        const uint32_t keep = valid >= uint32_t(lo + 4) ? 0xffffffffu
                                              : valid <= uint32_t(lo) ? 0u
                                              : (1u << (8 * (valid - lo))) - 1u;
                        out[w] &= keep;
                    }
                }
                x[0] = out[0]; x[1] = out[1]; x[2] = out[2]; x[3] = out[3];
            } else {
                x[0] = in[0]; x[1] = in[1]; x[2] = in[2]; x[3] = in[3];
            }
        }
    } else if (i < int64_t(sch.a)) {
        const uint32_t valid = uint32_t(i) == sch.a - 1 ? aad_tail : 16u;
        load_block<false>(v.aad + 16 * i, valid, x);
    } else {
        // length block [len(A)]_64 || [len(C)]_64 in bits, big-endian
        const uint64_t abits = uint64_t(sch.aad_bytes) * 8u;
        const uint64_t cbits = sch.bytes * 8u;
        x[0] = bswap32(uint32_t(abits >> 32));
        x[1] = bswap32(uint32_t(abits));
        x[2] = bswap32(uint32_t(cbits >> 32));
        x[3] = bswap32(uint32_t(cbits));
    }
    y[0] ^= x[0]; y[1] ^= x[1]; y[2] ^= x[2]; y[3] ^= x[3];
}

// Keystream of ciphertext block k (cached rounds 1-2 when allowed).
template <bool kCached>
__device__ __forceinline__ void keystream_block(const uint32_t* aes, AesLane lane, const AesKeys& keys,
                                                const CtrCache& cc, uint32_t n0, uint32_t n1,
                                                uint32_t n2, uint32_t ctr, uint32_t ks[4])
{
    if (kCached) aes_ctr_block_cached(aes, lane, keys, cc, ctr, ks);
    else aes_ctr_block(aes, lane, keys, n0, n1, n2, ctr, ks);
}

// Full-ciphertext rows [j0, j1) of this thread, two rows per step.  The
// loads of the next pair are issued before the current pair's keystreams are
// computed (software pipelining), so HBM latency hides behind the AES work.
// Rows of the fast region whose data is already loaded: straight-line code
// (no branches), so the compiler interleaves the GHASH work with the
// independent AES work of every block.  Two rows fold into the accumulator as
// y <- y*H^2T ^ x_a*H^T ^ x_b: two independent table products instead of a
// dependent chain of two.
// Ciphertext of the previous row pair, folded into GHASH during the next
// pair's keystreams (encrypt: GHASH depends on the AES output).
struct PendPair {
    uint32_t a[4], b[4];
};

template <int kMode, bool kCached, int kRows>
__device__ __forceinline__ void rows_body(const RecView& v, __amdgpu_buffer_rsrc_t dst, const uint4* gh,
                                          const uint4* gh2, const uint32_t* aes, AesLane lane,
                                          const AesKeys& keys, const CtrCache& cc, uint32_t n0,
                                          uint32_t n1, uint32_t n2, const uint64_t (&k)[kRows],
                                          const uint4 (&in)[kRows], const uint4 (&ksin)[kRows],
                                          uint32_t y[4], PendPair& pend)
{
    static_assert(kRows == 1 || kRows == 2, "rows per step");
    if constexpr (kRows == 2 && kCached && kMode == MODE_ENCRYPT) {
        // GHASH of the previous pair's ciphertext rides along with this
        // pair's keystreams.
        uint32_t ka[4], kb[4], acc[4];
        ctr2_ghash2(aes, lane, keys, cc, v.iv[3] + uint32_t(k[0]), v.iv[3] + uint32_t(k[1]), gh, gh2,
                    y, pend.a, ka, kb, acc);
        y[0] = acc[0] ^ pend.b[0]; y[1] = acc[1] ^ pend.b[1];
        y[2] = acc[2] ^ pend.b[2]; y[3] = acc[3] ^ pend.b[3];
        pend.a[0] = in[0].x ^ ka[0]; pend.a[1] = in[0].y ^ ka[1];
        pend.a[2] = in[0].z ^ ka[2]; pend.a[3] = in[0].w ^ ka[3];
        pend.b[0] = in[1].x ^ kb[0]; pend.b[1] = in[1].y ^ kb[1];
        pend.b[2] = in[1].z ^ kb[2]; pend.b[3] = in[1].w ^ kb[3];
        st_wt(dst, k[0], make_uint4(pend.a[0], pend.a[1], pend.a[2], pend.a[3]));
        st_wt(dst, k[1], make_uint4(pend.b[0], pend.b[1], pend.b[2], pend.b[3]));
        return;
    }
    if constexpr (kRows == 2 && kCached && kMode == MODE_DECRYPT) {
        // GHASH reads ciphertext only, so it interleaves with the keystreams.
        const uint32_t xa[4] = {in[0].x, in[0].y, in[0].z, in[0].w};
        uint32_t ka[4], kb[4], acc[4];
        ctr2_ghash2(aes, lane, keys, cc, v.iv[3] + uint32_t(k[0]), v.iv[3] + uint32_t(k[1]), gh, gh2,
                    y, xa, ka, kb, acc);
        y[0] = acc[0] ^ in[1].x; y[1] = acc[1] ^ in[1].y; y[2] = acc[2] ^ in[1].z; y[3] = acc[3] ^ in[1].w;
        st_wt(dst, k[0], make_uint4(in[0].x ^ ka[0], in[0].y ^ ka[1], in[0].z ^ ka[2], in[0].w ^ ka[3]));
        st_wt(dst, k[1], make_uint4(in[1].x ^ kb[0], in[1].y ^ kb[1], in[1].z ^ kb[2], in[1].w ^ kb[3]));
        return;
    }
    uint32_t s[kRows][4];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        if (kMode == MODE_VERIFY_XOR) {
            s[r][0] = ksin[r].x; s[r][1] = ksin[r].y; s[r][2] = ksin[r].z; s[r][3] = ksin[r].w;
        } else if (kMode != MODE_VERIFY) {
            keystream_block<kCached>(aes, lane, keys, cc, n0, n1, n2, v.iv[3] + uint32_t(k[r]), s[r]);
        }
    }
    uint4 o[kRows];
    uint32_t x[kRows][4];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        o[r] = in[r];
        if (kMode != MODE_VERIFY)
            o[r] = make_uint4(in[r].x ^ s[r][0], in[r].y ^ s[r][1], in[r].z ^ s[r][2], in[r].w ^ s[r][3]);
        const uint4 xv = kMode == MODE_ENCRYPT ? o[r] : in[r];
        x[r][0] = xv.x; x[r][1] = xv.y; x[r][2] = xv.z; x[r][3] = xv.w;
    }
    if (kRows == 2) {
        uint32_t a[4], b[4];
        gh_mul(gh2, y, a);
        gh_mul(gh, x[0], b);
#pragma unroll
        for (int w = 0; w < 4; ++w) y[w] = xor3(a[w], b[w], x[kRows - 1][w]);
    } else {
        gh_mul_table(gh, y);
#pragma unroll
        for (int w = 0; w < 4; ++w) y[w] ^= x[0][w];
    }
    if (kMode != MODE_VERIFY) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) st_wt(dst, k[r], o[r]);
    }
}

template <int kMode, int kRows>
__device__ __forceinline__ void load_rows(const uint4* __restrict__ src, const uint4* __restrict__ ksrc,
                                          const uint64_t (&k)[kRows], uint4 (&in)[kRows],
                                          uint4 (&ksin)[kRows])
{
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        in[r] = src[k[r]];
        if (kMode == MODE_VERIFY_XOR) ksin[r] = ksrc[k[r]];
    }
}

// Full-ciphertext rows [j0, j1) of this thread, two rows per step.  Ping-pong
// buffers: the loads of the next step are issued before the current step's
// keystreams, so HBM latency hides behind the AES work.
template <int kMode, bool kCached>
__device__ __forceinline__ void rows_fast(const RecView& v, const uint4* gh, const uint4* gh2,
                                          const uint32_t* aes, AesLane lane, const AesKeys& keys,
                                          const CtrCache& cc, uint32_t n0, uint32_t n1, uint32_t n2,
                                          uint64_t k0, uint32_t j0, uint32_t j1, uint32_t y[4])
{
    constexpr int kP = 2;
    const uint4* __restrict__ src = reinterpret_cast<const uint4*>(v.src);
    const uint4* __restrict__ ksrc = reinterpret_cast<const uint4*>(v.ks);
    const __amdgpu_buffer_rsrc_t dst = rsrc_of(v.dst);
    const uint32_t nsteps = (j1 - j0) / kP;
    const uint32_t jend = j0 + nsteps * kP;
    if (nsteps) {
        auto rows_of = [&](uint32_t step, uint64_t (&k)[kP]) {
            const uint32_t s = step < nsteps ? step : nsteps - 1;  // clamped prefetch
#pragma unroll
            for (int r = 0; r < kP; ++r) k[r] = k0 + uint64_t(j0 + s * kP + r) * SI_T;
        };
        // Encrypt folds each pair's ciphertext into GHASH during the next
        // pair, so its first pair only makes keystreams.
        constexpr bool kDelay = kMode == MODE_ENCRYPT && kCached;
        PendPair pend;
        uint32_t st0 = 0;
        if (kDelay) {
            uint64_t k2[kP];
            rows_of(0, k2);
            const uint4 p0 = src[k2[0]], p1 = src[k2[1]];
            uint32_t s0[4], s1[4];
            keystream_block<true>(aes, lane, keys, cc, n0, n1, n2, v.iv[3] + uint32_t(k2[0]), s0);
            keystream_block<true>(aes, lane, keys, cc, n0, n1, n2, v.iv[3] + uint32_t(k2[1]), s1);
            pend.a[0] = p0.x ^ s0[0]; pend.a[1] = p0.y ^ s0[1]; pend.a[2] = p0.z ^ s0[2]; pend.a[3] = p0.w ^ s0[3];
            pend.b[0] = p1.x ^ s1[0]; pend.b[1] = p1.y ^ s1[1]; pend.b[2] = p1.z ^ s1[2]; pend.b[3] = p1.w ^ s1[3];
            st_wt(dst, k2[0], make_uint4(pend.a[0], pend.a[1], pend.a[2], pend.a[3]));
            st_wt(dst, k2[1], make_uint4(pend.b[0], pend.b[1], pend.b[2], pend.b[3]));
            st0 = 1;
        }
        if (st0 < nsteps) {
            uint64_t ka[kP], kb[kP];
            uint4 a[kP], qa[kP], b[kP], qb[kP];
            rows_of(st0, ka);
            load_rows<kMode, kP>(src, ksrc, ka, a, qa);
            for (uint32_t st = st0; st < nsteps; st += 2) {
                rows_of(st + 1, kb);
                load_rows<kMode, kP>(src, ksrc, kb, b, qb);
                __builtin_amdgcn_sched_barrier(0);
                rows_body<kMode, kCached, kP>(v, dst, gh, gh2, aes, lane, keys, cc, n0, n1, n2, ka, a, qa, y, pend);
                if (st + 1 >= nsteps) break;
                rows_of(st + 2, ka);
                load_rows<kMode, kP>(src, ksrc, ka, a, qa);
                __builtin_amdgcn_sched_barrier(0);
                rows_body<kMode, kCached, kP>(v, dst, gh, gh2, aes, lane, keys, cc, n0, n1, n2, kb, b, qb, y, pend);
            }
        }
        if (kDelay) {
            uint32_t u[4], w4[4];
            gh_mul(gh2, y, u);
            gh_mul(gh, pend.a, w4);
#pragma unroll
            for (int w = 0; w < 4; ++w) y[w] = xor3(u[w], w4[w], pend.b[w]);
        }
    }
    for (uint32_t j = jend; j < j1; ++j) {
        uint64_t k1[1] = {k0 + uint64_t(j) * SI_T};
        uint4 a1[1], q1[1];
        load_rows<kMode, 1>(src, ksrc, k1, a1, q1);
        PendPair none;
        rows_body<kMode, kCached, 1>(v, dst, gh, gh2, aes, lane, keys, cc, n0, n1, n2, k1, a1, q1, y, none);
    }
}

// Rows [q0, q1) of one record: Horner with H^T over the thread's blocks into
// y.  Row q holds blocks m - (R - q)*T + t (row R-1 ends with the length
// block).  The owner of the length block also returns the tag mask E_K(J0).
template <int kMode, bool kAligned, bool kWT>
__device__ __forceinline__ void segment_rows(const GcmCtx* __restrict__ ctx, const RecBatch& batch,
                                             const Sched& sch, const RecView& v, const uint4* gh,
                                             const uint4* gh2, const uint32_t* aes, AesLane lane,
                                             const AesKeys& keys, uint32_t tid, uint32_t q0,
                                             uint32_t q1, uint32_t y[4], uint32_t ek[4])
{
    const uint32_t n0 = bswap32(v.iv[0]) ^ ctx->rk[0];
    const uint32_t n1 = bswap32(v.iv[1]) ^ ctx->rk[1];
    const uint32_t n2 = bswap32(v.iv[2]) ^ ctx->rk[2];
    const int64_t m = int64_t(sch.a) + int64_t(sch.n) + 1;
    const int64_t base = m - int64_t(sch.rows - q0) * SI_T;
    const uint32_t J = q1 - q0;
    const uint32_t tail = uint32_t(sch.bytes - (uint64_t(sch.n) - 1) * 16u);  // bytes in last block
    const uint32_t aad_tail = sch.aad_bytes ? uint32_t(sch.aad_bytes - (uint64_t(sch.a) - 1) * 16u) : 0u;

    // Rows whose blocks are all full ciphertext blocks for every thread of
    // the workgroup take the fast path: i in [a, a + nfull) for all t.
    const int64_t nfull = int64_t(sch.bytes / 16);
    int64_t jf0 = int64_t(sch.a) - base;                      // first fast row: base + j*T >= a
    jf0 = jf0 <= 0 ? 0 : (jf0 + SI_T - 1) / SI_T;
    int64_t jf1 = int64_t(sch.a) + nfull - base - SI_T;      // last fast row: base + j*T + T-1 < a + nfull
    jf1 = jf1 < 0 ? 0 : jf1 / SI_T + 1;
    if (jf1 > int64_t(J)) jf1 = J;
    if (jf0 > jf1) jf0 = jf1;
    const bool fast_ok = kAligned && !(v.bad && !batch.staging);
    if (!fast_ok) jf0 = jf1 = J;

    y[0] = y[1] = y[2] = y[3] = 0;
    for (uint32_t j = 0; j < uint32_t(jf0); ++j) {
        if (j != 0) gh_mul_table(gh, y);
        row_general<kMode, kAligned, kWT>(batch, sch, v, aes, lane, keys, n0, n1, n2,
                                          base + int64_t(j) * SI_T + tid, tail, aad_tail, y);
    }
    if (jf1 > jf0) {
        // Drain the key / descriptor loads so the loop's memory waits only
        // track the ciphertext stream.
        __builtin_amdgcn_s_waitcnt(0);
        const uint64_t k0 = uint64_t(base + tid - int64_t(sch.a));  // block of row 0 (may wrap; rows >= jf0 are valid)
        // Counter bytes 12..13 constant over the fast rows of the whole workgroup?
        const uint32_t clo = v.iv[3] + uint32_t(base + jf0 * SI_T - int64_t(sch.a));
        const uint32_t chi = v.iv[3] + uint32_t(base + jf1 * SI_T - 1 - int64_t(sch.a));
        const bool cached = (kMode == MODE_DECRYPT || kMode == MODE_ENCRYPT) && chi >= clo &&
                            (clo >> 16) == (chi >> 16);
        if (cached) {
            const uint32_t s3 = bswap32(v.iv[3] + uint32_t(k0 + uint64_t(jf0) * SI_T)) ^ keys.rk3;
            const CtrCache cc = ctr_cache(aes, lane, ctx, n0, n1, n2, s3);
            rows_fast<kMode, true>(v, gh, gh2, aes, lane, keys, cc, n0, n1, n2, k0, uint32_t(jf0),
                                   uint32_t(jf1), y);
        } else {
            const CtrCache cc{};
            rows_fast<kMode, false>(v, gh, gh2, aes, lane, keys, cc, n0, n1, n2, k0, uint32_t(jf0),
                                    uint32_t(jf1), y);
        }
    }
    for (uint32_t j = uint32_t(jf1); j < J; ++j) {
        if (j != 0) gh_mul_table(gh, y);
        row_general<kMode, kAligned, kWT>(batch, sch, v, aes, lane, keys, n0, n1, n2,
                                          base + int64_t(j) * SI_T + tid, tail, aad_tail, y);
    }
    ek[0] = ek[1] = ek[2] = ek[3] = 0;
    if (q1 == sch.rows && tid == SI_T - 1) aes_ctr_block(aes, lane, keys, n0, n1, n2, 1u, ek);
}

// Workgroup w = r*K + c owns rows [c*R/K, (c+1)*R/K) of record r (K chunks
// per record, chosen by the host so that the grid fills two workgroups per
// CU without a chunk ever spanning two records).
template <int kMode, bool kAligned, bool kWT>
__global__ __launch_bounds__(SI_T) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gcm_records_kernel(const GcmCtx* __restrict__ ctx, RecBatch batch, Sched sch,
                        RecAcc* __restrict__ acc)
{
    // Exactly 80 KiB so two workgroups share a CU:
    // [0, 8 KiB) GHASH tables of H^T, [8, 16 KiB) of H^2T, [16, 80 KiB) AES
    // Te0/Te1 copies.  After the row work the AES region holds the per-lane
    // tables of the placement multiply and the H^T region the reduction.
    __shared__ uint4 s_lds[1024 + 4096];
    uint4* const gh = s_lds;
    uint4* const gh2 = s_lds + 512;
    uint32_t* const aes = reinterpret_cast<uint32_t*>(s_lds + 1024);
    uint32_t(*const s_red)[4] = reinterpret_cast<uint32_t(*)[4]>(s_lds);
    uint32_t* const s_last = reinterpret_cast<uint32_t*>(s_lds + SI_T / 64);

    constexpr bool kNeedRelease = (kMode == MODE_DECRYPT || kMode == MODE_VERIFY_XOR) && !kWT;
    const uint32_t tid = threadIdx.x;
    {
        // Every global load of the set-up is issued before the first LDS
        // write, so the whole fill costs about one L2 round trip.
        const uint4 g0 = ctx->gh4[tid], g1 = ctx->gh4[tid + SI_T];
        const uint4 g2 = ctx->gh4b[tid], g3 = ctx->gh4b[tid + SI_T];
        aes_fill_lds(aes, ctx->te0, tid);
        gh[tid] = g0; gh[tid + SI_T] = g1;
        gh2[tid] = g2; gh2[tid + SI_T] = g3;
    }
    AesKeys keys;
    load_keys(ctx, keys);
    __syncthreads();

    const uint32_t r = blockIdx.x / sch.k;
    const uint32_t c = blockIdx.x % sch.k;
    const uint32_t q0 = uint32_t(uint64_t(c) * sch.rows / sch.k);
    const uint32_t q1 = uint32_t(uint64_t(c + 1) * sch.rows / sch.k);
    const RecView v = view_of(batch, r);
    uint32_t y[4], ek[4];
    segment_rows<kMode, kAligned, kWT>(ctx, batch, sch, v, gh, gh2, aes, aes_lane(tid & 63u), keys, tid,
                                       q0, q1, y, ek);
    __syncthreads();  // AES and GHASH tables are dead from here on

    // Thread t's partial covers blocks whose last one has exponent
    // (R - q1)*T + T - t; threads whose blocks all precede X carry zero.
    uint32_t q[4] = {0, 0, 0, 0};
    {
        const int64_t m = int64_t(sch.a) + int64_t(sch.n) + 1;
        const int64_t i_last = m - int64_t(sch.rows - q1 + 1) * SI_T + tid;
        const uint64_t e = i_last >= 0 ? uint64_t(sch.rows - q1) * SI_T + SI_T - tid : 0u;
        const uint4 zp = reinterpret_cast<const uint4*>(ctx + 1)[e];
        const uint32_t z[4] = {zp.x, zp.y, zp.z, zp.w};
        gh_mul_generic(y, z, reinterpret_cast<uint4*>(aes), tid, SI_T, q);
    }
    q[0] ^= ek[0]; q[1] ^= ek[1]; q[2] ^= ek[2]; q[3] ^= ek[3];
    wave_xor4(q);
    // Every wave's data stores must be complete (write-through) or at least
    // in L2 (before thread 0's release) when the ticket is taken; s_barrier
    // does not wait for them.
    __builtin_amdgcn_s_waitcnt(0);
    if ((tid & 63u) == 0) {
        s_red[tid >> 6][0] = q[0]; s_red[tid >> 6][1] = q[1];
        s_red[tid >> 6][2] = q[2]; s_red[tid >> 6][3] = q[3];
    }
    __syncthreads();
    RecAcc* ra = acc + r;
    if (tid == 0) {
        uint32_t t[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < SI_T / 64; ++w)
#pragma unroll
            for (int k = 0; k < 4; ++k) t[k] ^= s_red[w][k];
        if (sch.k == 1) {
            s_red[0][0] = t[0]; s_red[0][1] = t[1]; s_red[0][2] = t[2]; s_red[0][3] = t[3];
            *s_last = 1;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                __hip_atomic_fetch_xor(&ra->w[k], t[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // Take a ticket once this workgroup's data stores and XORs are
            // performed.  Write-through stores are complete after s_waitcnt;
            // byte-granular stores need the agent-scope release (L2 write-back).
            uint32_t prev;
            if (kNeedRelease) {
                prev = __hip_atomic_fetch_add(&ra->count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __builtin_amdgcn_s_waitcnt(0);
                prev = __hip_atomic_fetch_add(&ra->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            *s_last = prev == sch.k - 1 ? 1u : 0u;
            if (*s_last) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    s_red[0][k] = __hip_atomic_exchange(&ra->w[k], 0u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&ra->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    __syncthreads();
    if (!*s_last) return;
    
    // Finalise the record.
    if (kMode == MODE_ENCRYPT) {
        if (tid == 0 && v.bad && batch.fail_count) atomicAdd(batch.fail_count, 1u);
        if (tid < 4) {
            const uint32_t w = s_red[0][tid];
            for (int b = 0; b < 4; ++b) v.tag[4 * tid + b] = uint8_t(w >> (8 * b));
        }
        return;
    }
    uint32_t diff = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) diff |= uint32_t(uint8_t(s_red[0][k >> 2] >> (8 * (k & 3))) ^ v.tag[k]);
    const uint32_t ok = (diff == 0 && !v.bad) ? 1u : 0u;
    if (tid == 0) {
        *v.status = ok;
        if (!ok && batch.fail_count) atomicAdd(batch.fail_count, 1u);
    }
    if (!ok && kMode != MODE_VERIFY && !(v.bad && !batch.staging)) zero_bytes(v.dst, sch.bytes, tid, SI_T);
}

__global__ __launch_bounds__(SI_T) void ctr_kernel(const GcmCtx* __restrict__ ctx,
                                                   const uint8_t* __restrict__ in,
                                                   uint8_t* __restrict__ out, uint64_t bytes,
                                                   uint4 iv, int aligned)
{
    __shared__ uint32_t s_aes[256 * 64];
    const uint32_t tid = threadIdx.x;
    aes_fill_lds(s_aes, ctx->te0, tid);
    AesKeys keys;
    load_keys(ctx, keys);
    __syncthreads();
    const AesLane lane = aes_lane(tid & 63u);
    const uint32_t n0 = bswap32(iv.x) ^ ctx->rk[0];
    const uint32_t n1 = bswap32(iv.y) ^ ctx->rk[1];
    const uint32_t n2 = bswap32(iv.z) ^ ctx->rk[2];
    const uint64_t nb = (bytes + 15) / 16;
    for (uint64_t k = uint64_t(blockIdx.x) * SI_T + tid; k < nb; k += uint64_t(gridDim.x) * SI_T) {
        const uint32_t valid = k == nb - 1 ? uint32_t(bytes - 16 * k) : 16u;
        uint32_t ks[4], d[4] = {0, 0, 0, 0};
        aes_ctr_block(s_aes, lane, keys, n0, n1, n2, iv.w + uint32_t(k), ks);
        if (in) {
            if (aligned) load_block<true>(in + 16 * k, valid, d);
            else load_block<false>(in + 16 * k, valid, d);
        }
        const uint32_t o[4] = {d[0] ^ ks[0], d[1] ^ ks[1], d[2] ^ ks[2], d[3] ^ ks[3]};
        if (aligned) store_block<true>(out + 16 * k, valid, o);
        else store_block<false>(out + 16 * k, valid, o);
    }
}

__global__ void auth_gate_kernel(uint8_t* data, const uint32_t* status, uint64_t bytes)
{
    if (*status == 1u) return;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride)
        data[i] = 0;
}

// ---------------------------------------------------------------- launches

template <int kMode>
static hipError_t launch_mode(hipStream_t stream, const GcmCtx* ctx, const RecBatch& b,
                              const Sched& s, RecAcc* acc, bool aligned)
{
    const dim3 grid(s.nrec * s.k), block(SI_T);
    if (aligned && s.bytes % 16 == 0)
        hipLaunchKernelGGL((gcm_records_kernel<kMode, true, true>), grid, block, 0, stream, ctx, b, s, acc);
    else if (aligned)
        hipLaunchKernelGGL((gcm_records_kernel<kMode, true, false>), grid, block, 0, stream, ctx, b, s, acc);
    else
        hipLaunchKernelGGL((gcm_records_kernel<kMode, false, false>), grid, block, 0, stream, ctx, b, s, acc);
    return hipGetLastError();
}

hipError_t launch_gcm(int mode, hipStream_t stream, const GcmCtx* ctx, const RecBatch& b,
                      const Sched& s, RecAcc* acc, bool aligned)
{
    switch (mode) {
    case MODE_DECRYPT: return launch_mode<MODE_DECRYPT>(stream, ctx, b, s, acc, aligned);
    case MODE_ENCRYPT: return launch_mode<MODE_ENCRYPT>(stream, ctx, b, s, acc, aligned);
    case MODE_VERIFY: return launch_mode<MODE_VERIFY>(stream, ctx, b, s, acc, aligned);
    case MODE_VERIFY_XOR: return launch_mode<MODE_VERIFY_XOR>(stream, ctx, b, s, acc, aligned);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_ctr(hipStream_t stream, const GcmCtx* ctx, const uint8_t* in, uint8_t* out,
                      uint64_t bytes, const uint32_t iv[4])
{
    const uint64_t nb = (bytes + 15) / 16;
    uint64_t grid = (nb + SI_T - 1) / SI_T;
    if (grid > 4096) grid = 4096;
    const bool aligned = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
    hipLaunchKernelGGL(ctr_kernel, dim3(uint32_t(grid)), dim3(SI_T), 0, stream, ctx, in, out, bytes,
                       make_uint4(iv[0], iv[1], iv[2], iv[3]), aligned ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_auth_gate(hipStream_t stream, uint8_t* data, const uint32_t* status, uint64_t bytes)
{
    uint64_t grid = (bytes + 255) / 256;
    if (grid > 1024) grid = 1024;
    if (grid == 0) grid = 1;
    hipLaunchKernelGGL(auth_gate_kernel, dim3(uint32_t(grid)), dim3(256), 0, stream, data, status, bytes);
    return hipGetLastError();
}

}  // namespace si
