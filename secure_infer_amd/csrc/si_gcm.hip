// AES-128-GCM record kernels for gfx950.
//
// One launch processes a batch of records.  Each record's GHASH input is the
// block sequence X = AAD || C || L (SP 800-38D), m = a + n + 1 blocks, and
// GHASH = XOR_k X_k * H^(m-k).  AAD || C (m - 1 blocks) is cut into R rows
// of T = 256 blocks counted from its end (row R-1 ends with the last
// ciphertext block; row 0 may start before X); the length block L adds L * H,
// the same for every record of a batch (passed in by the host).  A
// workgroup of three 256-thread units takes a contiguous share of the
// records' concatenated rows (laid out by the host; one or two records);
// thread t of a unit owns block t of each of its rows, so every row is one
// coalesced 4 KiB sweep, and the units interleave the share's rows.  Per
// thread:
//   * CTR: keystream of counter iv3 + k for ciphertext block k (32-bit wrap,
//     ghash.aicpu:174-221), XORed into the data and stored;
//   * GHASH: Horner with H^768 over the unit's rows (LDS tables), a move onto
//     the segment's exponent grid (H^256 or H^512), and a placement multiply
//     by H^((R - qb)*T + T - t) (qb = end row of the segment) shared by the
//     SI_U threads of position t.
// Partials are XOR-reduced over the workgroup and then across workgroups with
// device-scope atomics; a row count names the workgroup that completes a
// record, which compares the tag in constant time, writes the status and, on
// failure, zeroes the record's output before the kernel ends.
// The zeroing must land after every plaintext store of the record:
// full-block stores are issued write-through (sc1, agent-coherent) and
// drained (s_waitcnt) before a workgroup takes its ticket; byte-granular
// stores (partial or unaligned blocks) fall back to an agent-scope release
// (L2 write-back) instead.
#include <map>
#include <mutex>

#include "si_device.h"
#include "si_clock.h"
#include "si_kernels.h"

namespace si {

// The allocation-free reload's scratch: one array per GPU, held until the
// process ends.  Host code never uses the array's name as an address (on the
// host it is a stand-in, not a device address): noalloc_scratch() looks the
// address up per device with hipGetSymbolAddress and every kernel argument
// derives from that.
static __device__ __align__(256) uint8_t scratch[SI_NOALLOC_SCRATCH_BYTES];
static_assert(sizeof(RecAcc) == 32, "accumulator region holds 32 B per record");

enum Mode : int {
    MODE_DECRYPT = 0,     // verify + decrypt, output zeroed on failure
    MODE_ENCRYPT = 1,     // encrypt + tag
    MODE_VERIFY = 2,      // tag check only
    MODE_VERIFY_XOR = 3,  // verify + XOR with a given keystream
};

// Record buffers are device (global) memory.  The record views are rebuilt
// from LDS words, which loses that fact; accessing them through generic
// pointers would emit FLAT instructions, which also count on the LDS wait
// counter and so force the LDS pipeline to drain behind every HBM access.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p)
{
    return (const __attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gmem(T* p)
{
    return (__attribute__((address_space(1))) T*)p;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 gload4(const void* p)
{
    const u32x4 v = *gmem(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void gstore4(void* p, uint4 w)
{
    u32x4 v;
    v.x = w.x; v.y = w.y; v.z = w.z; v.w = w.w;
    *gmem(reinterpret_cast<u32x4*>(p)) = v;
}

template <bool kAligned>
__device__ __forceinline__ void load_block(const uint8_t* p, uint32_t valid, uint32_t w[4])
{
    if (kAligned && valid == 16u) {
        const uint4 v = gload4(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        return;
    }
    w[0] = w[1] = w[2] = w[3] = 0;
    const auto* g = gmem(p);
    for (uint32_t b = 0; b < valid; ++b) w[b >> 2] |= uint32_t(g[b]) << (8 * (b & 3));
}

template <bool kAligned>
__device__ __forceinline__ void store_block(uint8_t* p, uint32_t valid, const uint32_t w[4])
{
    if (kAligned && valid == 16u) {
        gstore4(p, make_uint4(w[0], w[1], w[2], w[3]));
        return;
    }
    auto* g = gmem(p);
    for (uint32_t b = 0; b < valid; ++b) g[b] = uint8_t(w[b >> 2] >> (8 * (b & 3)));
}

__device__ __forceinline__ void zero_bytes(uint8_t* p, uint64_t bytes, uint32_t tid,
                                           uint32_t nthreads)
{
    const bool aligned = (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
    auto* g = gmem(p);
    if (aligned) {
        const uint64_t full = bytes >> 4;
        for (uint64_t i = tid; i < full; i += nthreads) gstore4(p + 16 * i, make_uint4(0, 0, 0, 0));
        for (uint64_t i = (full << 4) + tid; i < bytes; i += nthreads) g[i] = 0;
    } else {
        for (uint64_t i = tid; i < bytes; i += nthreads) g[i] = 0;
    }
}

// Everything the kernel body needs about one record (80 bytes, kept in LDS
// so the batch's kernel arguments are dead after the set-up).
struct RecView {
    const uint8_t* src;  // ciphertext (decrypt/verify) or plaintext (encrypt)
    uint8_t* dst;        // plaintext out (decrypt) or ciphertext out (encrypt)
    const uint8_t* aad;
    uint8_t* tag;        // expected tag, or tag output (encrypt)
    uint32_t* status;
    const uint8_t* ks;   // keystream (verify_xor)
    uint32_t* fail_count;
    uint32_t iv[4];
    uint32_t bad;        // block-table entry out of range: the record fails
    uint32_t skip;       // bad and no staging: touch no cache memory
};
static_assert(sizeof(RecView) == 80, "five 16-byte LDS words");

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
        v.fail_count = b.fail_count;
        v.bad = v.skip = 0;
        return v;
    }
    uint8_t* wire = const_cast<uint8_t*>(b.wire) + uint64_t(r) * b.wire_stride;
    const uint32_t kind = r < b.n_k ? 0u : 1u;
    const int64_t sid = b.slots[r];
    v.bad = (sid < 0 || sid >= b.nslots) ? 1u : 0u;
    v.skip = v.bad && !b.staging ? 1u : 0u;
    v.fail_count = b.fail_count;
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

// One general row: any mix of padding, AAD and ciphertext blocks, partial
// blocks and unaligned buffers.  Used for the rows at a record's ends.  When
// ek_dst is given (the record's row 0), the lane of AAD block a-1 forms the
// tag mask E_K(J0) (counter 1) in the same keystream pass as the ciphertext
// lanes and stores it there.
template <int kMode, bool kAligned, bool kWT>
__device__ __forceinline__ void row_general(const Sched& sch, const RecView& v,
                                            const uint32_t* aes, AesLane lane, const AesKeys& keys,
                                            uint32_t n0, uint32_t n1, uint32_t n2, int64_t i,
                                            uint32_t tail, uint32_t aad_tail, uint4* ek_dst,
                                            uint32_t y[4])
{
    if (i < 0) return;
    const bool ct = i >= int64_t(sch.a) && i < int64_t(sch.a) + int64_t(sch.n);
    const bool ek = ek_dst != nullptr && i == int64_t(sch.a) - 1;
    if (ct && v.skip) return;
    const uint64_t k = ct ? uint64_t(i - sch.a) : 0u;
    uint32_t ks[4] = {0, 0, 0, 0};
    if ((ct && (kMode == MODE_DECRYPT || kMode == MODE_ENCRYPT)) || ek)
        aes_ctr_block(aes, lane, keys, n0, n1, n2, ek ? 1u : v.iv[3] + uint32_t(k), ks);
    if (ek) *ek_dst = make_uint4(ks[0], ks[1], ks[2], ks[3]);
    uint32_t x[4];
    if (ct) {
        const uint32_t valid = k == uint64_t(sch.n) - 1 ? tail : 16u;
        uint32_t in[4];
        load_block<kAligned>(v.src + 16 * k, valid, in);
        if (kMode == MODE_VERIFY) {
            x[0] = in[0]; x[1] = in[1]; x[2] = in[2]; x[3] = in[3];
        } else {
            if (kMode == MODE_VERIFY_XOR) load_block<kAligned>(v.ks + 16 * k, valid, ks);
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
        if ((reinterpret_cast<uintptr_t>(v.aad) & 15u) == 0)  // the wire record's AAD is
            load_block<true>(v.aad + 16 * i, valid, x);       // 32-byte aligned
        else
            load_block<false>(v.aad + 16 * i, valid, x);
    } else {
        return;  // past the ciphertext (the rows end with it)
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
// dependent chain of two.  Decrypt hashes the ciphertext it loaded while the
// keystreams are formed (the hand-pipelined pair step); encrypt hashes the
// ciphertext it has just made, after its keystreams.  (Encrypt folding each
// pair's ciphertext into the next pair's pipelined step measured slower on
// MI355X: 70B int4 writeback 86.2 vs 86.8 us per layer, ABBA on one GPU.)
template <int kMode, bool kCached, int kRows>
__device__ __forceinline__ void rows_body(const RecView& v, __amdgpu_buffer_rsrc_t dst, const uint4* gh,
                                          const uint4* gh2, const uint32_t* aes, AesLane lane,
                                          const AesKeys& keys, const CtrCache& cc, uint32_t n0,
                                          uint32_t n1, uint32_t n2, const uint64_t (&k)[kRows],
                                          const uint4 (&in)[kRows], const uint4 (&ksin)[kRows],
                                          uint32_t y[4])
{
    static_assert(kRows == 1 || kRows == 2, "rows per step");
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
        in[r] = gload4(src + k[r]);
        if (kMode == MODE_VERIFY_XOR) ksin[r] = gload4(ksrc + k[r]);
    }
}

// Issue priority of a wave with `left` pair steps to go (this one included).
// The arbiter otherwise favours the oldest wave: it runs one unit's rows to
// the end while the others wait, then leaves the last unit alone on the SIMDs
// with too few waves to hide latency.  Dropping a step's priority as a wave
// gets ahead keeps the units of a workgroup within about a step of each other.
__device__ __forceinline__ void step_priority(uint32_t left)
{
    if (left >= 4) __builtin_amdgcn_s_setprio(3);
    else if (left == 3) __builtin_amdgcn_s_setprio(2);
    else if (left == 2) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// Full-ciphertext rows i in [i0, i1) of this thread's unit (block k = kb +
// i*S, S = SI_U*SI_T), two rows per step.  Ping-pong buffers: the loads of
// the next step are issued before the current step's keystreams, so HBM
// latency hides behind the AES work.  Horner with gh = H^S, gh2 = H^2S.
template <int kMode, bool kCached>
__device__ __forceinline__ void rows_fast(const RecView& v, const uint4* gh, const uint4* gh2,
                                          const uint32_t* aes, AesLane lane, const AesKeys& keys,
                                          const CtrCache& cc, uint32_t n0, uint32_t n1, uint32_t n2,
                                          uint64_t kb, uint32_t i0, uint32_t i1, uint32_t y[4])
{
    constexpr int kP = 2;
    constexpr uint64_t kS = uint64_t(SI_U) * SI_T;
    const uint4* __restrict__ src = reinterpret_cast<const uint4*>(v.src);
    const uint4* __restrict__ ksrc = reinterpret_cast<const uint4*>(v.ks);
    const __amdgpu_buffer_rsrc_t dst = rsrc_of(v.dst);
    const uint32_t nsteps = (i1 - i0) / kP;
    const uint32_t iend = i0 + nsteps * kP;
    if (nsteps) {
        auto rows_of = [&](uint32_t step, uint64_t (&k)[kP]) {
            const uint32_t s = step < nsteps ? step : nsteps - 1;  // clamped prefetch
#pragma unroll
            for (int r = 0; r < kP; ++r) k[r] = kb + uint64_t(i0 + s * kP + r) * kS;
        };
        uint64_t ka[kP], kb2[kP];
        uint4 a[kP], qa[kP], b[kP], qb[kP];
        rows_of(0, ka);
        load_rows<kMode, kP>(src, ksrc, ka, a, qa);
        for (uint32_t st = 0; st < nsteps; st += 2) {
            rows_of(st + 1, kb2);
            load_rows<kMode, kP>(src, ksrc, kb2, b, qb);
            __builtin_amdgcn_sched_barrier(0);
            step_priority(nsteps - st);
            rows_body<kMode, kCached, kP>(v, dst, gh, gh2, aes, lane, keys, cc, n0, n1, n2, ka, a, qa, y);
            if (st + 1 >= nsteps) break;
            rows_of(st + 2, ka);
            load_rows<kMode, kP>(src, ksrc, ka, a, qa);
            __builtin_amdgcn_sched_barrier(0);
            step_priority(nsteps - st - 1);
            rows_body<kMode, kCached, kP>(v, dst, gh, gh2, aes, lane, keys, cc, n0, n1, n2, kb2, b, qb, y);
        }
        __builtin_amdgcn_s_setprio(0);
    }
    for (uint32_t i = iend; i < i1; ++i) {
        uint64_t k1[1] = {kb + uint64_t(i) * kS};
        uint4 a1[1], q1[1];
        load_rows<kMode, 1>(src, ksrc, k1, a1, q1);
        rows_body<kMode, kCached, 1>(v, dst, gh, gh2, aes, lane, keys, cc, n0, n1, n2, k1, a1, q1, y);
    }
}

// The fast rows of unit u in the segment rows [qa, qb): segment rows whose
// blocks are all full ciphertext blocks for every thread of a unit
// (i in [a, a + nfull) for all t), as the unit's row indices i in [i0, i1)
// (segment row u + SI_U*i), and the segment's first block (row 0).
struct FastRows {
    int64_t base;
    int64_t jf0, jf1;
    uint32_t nu, i0, i1;
};

__device__ __forceinline__ FastRows fast_rows(const Sched& sch, uint32_t u, uint32_t qa, uint32_t qb,
                                              bool fast_ok)
{
    FastRows f;
    const int64_t m = int64_t(sch.a) + int64_t(sch.n);  // AAD || C
    f.base = m - int64_t(sch.rows - qa) * SI_T;
    const uint32_t J = qb - qa;
    f.nu = u < J ? (J - u + SI_U - 1) / SI_U : 0u;
    const int64_t nfull = int64_t(sch.bytes / 16);
    int64_t jf0 = int64_t(sch.a) - f.base;                    // first fast row: base + j*T >= a
    jf0 = jf0 <= 0 ? 0 : (jf0 + SI_T - 1) / SI_T;
    int64_t jf1 = int64_t(sch.a) + nfull - f.base - SI_T;    // last fast row: base + j*T + T-1 < a + nfull
    jf1 = jf1 < 0 ? 0 : jf1 / SI_T + 1;
    if (jf1 > int64_t(J)) jf1 = J;
    if (jf0 > jf1) jf0 = jf1;
    if (!fast_ok) jf0 = jf1 = J;
    const auto first_at = [&](int64_t j) -> uint32_t {
        return j <= int64_t(u) ? 0u : uint32_t((j - int64_t(u) + SI_U - 1) / SI_U);
    };
    f.i1 = first_at(jf1);
    f.i0 = first_at(jf0);
    if (f.i1 > f.nu) f.i1 = f.nu;
    if (f.i0 > f.i1) f.i0 = f.i1;
    f.jf0 = jf0;
    f.jf1 = jf1;
    return f;
}

// Rows [qa, qb) of one record, shared by the workgroup's SI_U units: unit u
// takes the segment rows j = u + SI_U*i, i = 0..nu-1, and runs Horner with
// H^(SI_U*T) over them into y.  Row q of the record holds blocks
// m' - (R - q)*T + t of AAD || C (m' = a + n; row R-1 ends with the last
// ciphertext block).
template <int kMode, bool kAligned, bool kWT>
__device__ __forceinline__ void unit_rows(const GcmCtx* __restrict__ ctx, const Sched& sch, const RecView& v, const uint4* gh,
                                          const uint4* gh2, const uint32_t* aes, AesLane lane,
                                          const AesKeys& keys, uint32_t t, uint32_t u, uint32_t qa,
                                          uint32_t qb, uint4* ek_slot, uint32_t y[4])
{
    const uint32_t n0 = bswap32(v.iv[0]) ^ ctx->rk[0];
    const uint32_t n1 = bswap32(v.iv[1]) ^ ctx->rk[1];
    const uint32_t n2 = bswap32(v.iv[2]) ^ ctx->rk[2];
    const uint32_t tail = uint32_t(sch.bytes - (uint64_t(sch.n) - 1) * 16u);  // bytes in last block
    const uint32_t aad_tail = sch.aad_bytes ? uint32_t(sch.aad_bytes - (uint64_t(sch.a) - 1) * 16u) : 0u;
    const FastRows f = fast_rows(sch, u, qa, qb, kAligned && !v.skip);
    const int64_t base = f.base;
    const int64_t jf0 = f.jf0, jf1 = f.jf1;
    const uint32_t nu = f.nu, i0 = f.i0, i1 = f.i1;

    // Record row 0 (qa = 0: unit 0's first row; general, before or after the
    // fast rows) carries the tag-mask job when the batch puts it there.
    uint4* const ek_row = (sch.ek_row0 && qa == 0 && u == 0) ? ek_slot : nullptr;
    y[0] = y[1] = y[2] = y[3] = 0;
    for (uint32_t i = 0; i < i0; ++i) {
        if (i != 0) gh_mul_table(gh, y);
        row_general<kMode, kAligned, kWT>(sch, v, aes, lane, keys, n0, n1, n2,
                                          base + int64_t(u + SI_U * i) * SI_T + t, tail, aad_tail,
                                          i == 0 ? ek_row : nullptr, y);
    }
    if (i1 > i0) {
        // Drain the key / descriptor loads so the loop's memory waits only
        // track the ciphertext stream.
        __builtin_amdgcn_s_waitcnt(0);
        const uint64_t k0 = uint64_t(base + t - int64_t(sch.a));  // block of segment row 0 (may wrap; fast rows are valid)
        // Counter bytes 12..13 constant over the fast rows of all units?
        const uint32_t clo = v.iv[3] + uint32_t(base + jf0 * SI_T - int64_t(sch.a));
        const uint32_t chi = v.iv[3] + uint32_t(base + jf1 * SI_T - 1 - int64_t(sch.a));
        const bool cached = (kMode == MODE_DECRYPT || kMode == MODE_ENCRYPT) && chi >= clo &&
                            (clo >> 16) == (chi >> 16);
        const uint64_t kb = k0 + uint64_t(u) * SI_T;
        if (cached) {
            const uint32_t s3 = bswap32(v.iv[3] + uint32_t(kb + uint64_t(i0) * SI_U * SI_T)) ^ keys.rk3;
            const CtrCache cc = ctr_cache(aes, lane, ctx, n0, n1, n2, s3);
            rows_fast<kMode, true>(v, gh, gh2, aes, lane, keys, cc, n0, n1, n2, kb, i0, i1, y);
        } else {
            const CtrCache cc{};
            rows_fast<kMode, false>(v, gh, gh2, aes, lane, keys, cc, n0, n1, n2, kb, i0, i1, y);
        }
    }
    for (uint32_t i = i1; i < nu; ++i) {
        if (i != 0) gh_mul_table(gh, y);
        row_general<kMode, kAligned, kWT>(sch, v, aes, lane, keys, n0, n1, n2,
                                          base + int64_t(u + SI_U * i) * SI_T + t, tail, aad_tail,
                                          i == 0 ? ek_row : nullptr, y);
    }
}

// Placement multiplier of thread position t for a segment ending at row qb:
// H^((R - qb)*T + T - t + 1), the exponent of the thread's last block in the
// segment (+1: the length block follows the ciphertext); a thread whose
// blocks all precede X carries zero and takes H^0.
__device__ __forceinline__ uint4 placement_power(const GcmCtx* __restrict__ ctx, const Sched& sch,
                                                 uint32_t qb, uint32_t t)
{
    const int64_t m = int64_t(sch.a) + int64_t(sch.n);
    const int64_t l = m - int64_t(sch.rows - qb + 1) * SI_T + t;
    const uint64_t e = l >= 0 ? uint64_t(sch.rows - qb) * SI_T + SI_T - t + 1 : 0u;
    return reinterpret_cast<const uint4*>(ctx + 1)[e];
}

// Record view r of the batch -> LDS (five 16-byte words).
__device__ __forceinline__ void put_view(uint4* dst, const RecView& v)
{
    const uint4* w = reinterpret_cast<const uint4*>(&v);
#pragma unroll
    for (int i = 0; i < 5; ++i) dst[i] = w[i];
}

// LDS -> record view in scalar registers (the view is uniform).
__device__ __forceinline__ RecView get_view(const uint4* src)
{
    RecView v;
    uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const uint4 q = src[i];
        w[4 * i] = __builtin_amdgcn_readfirstlane(q.x);
        w[4 * i + 1] = __builtin_amdgcn_readfirstlane(q.y);
        w[4 * i + 2] = __builtin_amdgcn_readfirstlane(q.z);
        w[4 * i + 3] = __builtin_amdgcn_readfirstlane(q.w);
    }
    return v;
}

// The SI_U units' products of position t (xs[u*T + t]) XORed together.
__device__ __forceinline__ void unit_sum(const uint4* xs, uint32_t t, uint32_t out[4])
{
    static_assert(SI_U == 2 || SI_U == 3, "two or three units");
    const uint4 a = xs[t], b = xs[SI_T + t];
    const uint4 c = SI_U == 3 ? xs[2 * SI_T + t] : make_uint4(0, 0, 0, 0);
    out[0] = xor3(a.x, b.x, c.x); out[1] = xor3(a.y, b.y, c.y);
    out[2] = xor3(a.z, b.z, c.z); out[3] = xor3(a.w, b.w, c.w);
}

// Thread (u, t)'s part of the placement products of position t (the
// nibbles j = u mod SI_U; gh_mul_part).
template <int NS>
__device__ __forceinline__ void place_part(uint32_t u, const uint32_t (&x)[NS][4], const uint4* const (&tb)[NS],
                                           const uint4* zero, uint32_t t, uint32_t (&z)[NS][4])
{
    if (u == 0) gh_mul_part<SI_U, 0, NS>(x, tb, zero, t, SI_T, z);
    else if (u == 1 || SI_U == 2) gh_mul_part<SI_U, 1, NS>(x, tb, zero, t, SI_T, z);
    else gh_mul_part<SI_U, (SI_U == 3 ? 2 : 1), NS>(x, tb, zero, t, SI_T, z);
}

// Workgroup w owns a contiguous share of the records' concatenated row
// sequence (laid out by the host so that a share that straddles two records,
// which pays a second set of boundary rows and placements, takes fewer
// rows).  A share spans at most R rows (one or two segments), or, when the
// records outnumber the CUs, two whole records (a pair: two segments that
// both end at row R).
// Phases, separated by workgroup barriers:
//   1. rows: every unit runs its rows of each segment; its Horner partial is
//      multiplied by H^(d*T) (d = segment rows after the unit's last one, <
//      SI_U), which puts all units of a segment on the same exponent grid;
//   2. combine: the units that do not place a segment hand their products
//      to the one that does (unit s places segment s) through LDS;
//   3. placement: the placing thread t multiplies the sum by
//      H^((R - qb)*T + T - t) (qb = end row of the segment) from the power
//      table; wave XOR-reduction into LDS (the owner of the record's last
//      block adds the tag mask E_K(J0) there);
//   4. ticket: per segment, device atomics XOR the partial into the record's
//      accumulator and add the segment's rows to its row count; the
//      workgroup that completes R rows finalises the record.
template <int kMode, bool kAligned, bool kWT>
__device__ __forceinline__ void gcm_records_body(const GcmCtx* __restrict__ ctx, const RecBatch& batch,
                                                 const Sched& sch, RecAcc* __restrict__ acc)
{
    // 160 KiB, in 16-byte words.  During the rows:
    //   [0, 1024)      H^UT, H^2UT tables (row steps; below 64 KiB, so every
    //                  table read takes its offset as an immediate)
    //   [1024, 5120)   AES Te0/Te1 copies
    //   [5120, 6144)   H^T, H^2T tables (unit combine)
    // after them:
    //   [0, 768)       the units' products of the last segment
    //   [768, 783)     its wave sums, the record sums, last flags
    //   [1024, 4864)   placement table of segment 1 (straddling share), or
    //   [1024, 1792)   segment 0's products (pair)
    // throughout: [6144, 9984) the placement table of segment 0 (built in
    // the set-up; a straddling workgroup keeps segment 0's products and both
    // multipliers there until after the rows), 9984 a zero word, [9985, 9995) the two record views,
    // [9995, 9997) their tag masks E_K(J0), [9997, 10009) the wave sums of a
    // two-segment workgroup's segment 0, [10009, 10011) the expected tags.
    __shared__ uint4 s_lds[10240];
    const uint4* const g_u = s_lds;
    const uint4* const g_u2 = s_lds + 512;
    uint32_t* const aes = reinterpret_cast<uint32_t*>(s_lds + 1024);
    const uint4* const g_1 = s_lds + 5120;
    const uint4* const g_2 = s_lds + 5632;
    uint4* const xs = s_lds;
    uint4* const s_red = s_lds + 768;
    uint32_t(*const s_fin)[4] = reinterpret_cast<uint32_t(*)[4]>(s_lds + 768 + SI_NT / 64);
    uint32_t* const s_last = reinterpret_cast<uint32_t*>(s_lds + 768 + SI_NT / 64 + 2);
    uint4* const ptab1 = s_lds + 1024;
    uint4* const ptab0 = s_lds + 6144;
    uint4* const s_zp = s_lds + 6144 + SI_NT;  // straddling workgroups, during the rows
    uint4* const s_zero = s_lds + 9984;
    uint4* const s_view = s_lds + 9985;
    uint4* const s_ek = s_lds + 9995;
    uint4* const s_c0 = s_lds + 9997;
    uint4* const s_tag = s_lds + 10009;  // expected tags of the two records (decrypt, verify)
    uint4* const xs0 = s_lds + 1024;     // after the rows: a pair's segment-0 products

    constexpr bool kNeedRelease = (kMode == MODE_DECRYPT || kMode == MODE_VERIFY_XOR) && !kWT;
    // An allocation-free call that does not own the GPU's scratch touches
    // nothing; its finishing kernel fails every record closed.
    if (sch.gate && *gmem(sch.gate) == 0u) return;
    const uint32_t tid = threadIdx.x;
    // Unit index: uniform over a wave (SI_T is a multiple of 64).
    const uint32_t u = __builtin_amdgcn_readfirstlane(tid / SI_T), t = tid % SI_T;

    // The AES and GHASH tables depend on the key context only: their loads
    // go out first, in the shadow of the kernel-argument round trip that
    // gives this workgroup's share.  Every global load of the fill is issued
    // before its first LDS write, so it costs about one L2 round trip.
    if (tid < SI_T) {
        aes_fill_lds(aes, ctx->te0, tid);
    } else {
        // the 512 entries of each table over the other threads
        auto fill = [&](uint32_t i) {
            const uint4 a0 = ctx->gh4u[i], a1 = ctx->gh4u2[i], a2 = ctx->gh4[i], a3 = ctx->gh4b[i];
            s_lds[i] = a0;
            s_lds[512 + i] = a1;
            s_lds[5120 + i] = a2;
            s_lds[5632 + i] = a3;
        };
        if constexpr (SI_NT - SI_T == 512) fill(tid - SI_T);
        else
            for (uint32_t i = tid - SI_T; i < 512u; i += SI_NT - SI_T) fill(i);
    }

    // This workgroup's share of the records' concatenated rows.
    const uint64_t G = uint64_t(sch.nrec) * sch.rows;
    const uint64_t g0 = sch.use_starts ? sch.starts[blockIdx.x] : uint64_t(blockIdx.x) * G / sch.nwg;
    const uint64_t g1 = sch.use_starts ? sch.starts[blockIdx.x + 1] : (uint64_t(blockIdx.x) + 1) * G / sch.nwg;
    if (g1 == g0) return;  // an empty share (the whole workgroup: no barrier is pending)
    const uint32_t r0 = uint32_t(g0 / sch.rows);
    const uint32_t qa0 = uint32_t(g0 - uint64_t(r0) * sch.rows);
    const uint32_t qb0 = g1 - uint64_t(r0) * sch.rows < sch.rows ? uint32_t(g1 - uint64_t(r0) * sch.rows) : sch.rows;
    const uint32_t nseg = g1 > (uint64_t(r0) + 1) * sch.rows ? 2u : 1u;
    const uint32_t qb1 = uint32_t(g1 - (uint64_t(r0) + 1) * sch.rows);  // segment 1: rows [0, qb1) of r0 + 1
    // Two whole records (the host's pair layout): both segments end at row
    // R, so one placement table serves both.
    const bool pair = nseg == 2 && sch.pairs;

    // A one-segment workgroup's placement multiplier, loaded with the tables
    // below (its placement table is built in the set-up).
    // A straddling workgroup's two multipliers wait in LDS (after segment 0's
    // parked products) until its tables are built after the rows.
    uint4 zp0 = make_uint4(0, 0, 0, 0), zp1 = make_uint4(0, 0, 0, 0);
    zp0 = placement_power(ctx, sch, qb0, t);
    if (nseg == 2 && !pair && u == 0) zp1 = placement_power(ctx, sch, qb1, t);
    if (tid < nseg) put_view(s_view + 5 * tid, view_of(batch, r0 + tid));
    if (tid == 0) *s_zero = make_uint4(0, 0, 0, 0);
    // One segment or a pair: its placement table now (thread (u, t) writes
    // its third of the multiples of H^((R - qb)*T + T - t)).  Two segments
    // of a straddling share: the region holds segment 0's products while
    // segment 1 runs; both tables are built after the rows.
    if (nseg == 1 || pair) {
        const uint32_t z[4] = {zp0.x, zp0.y, zp0.z, zp0.w};
        gh_table_share<SI_U>(z, u, ptab0, t, SI_T);
    } else if (u == 0) {
        s_zp[t] = zp0;
        s_zp[SI_T + t] = zp1;
    }
    AesKeys keys;
    load_keys(ctx, keys);
    __syncthreads();
    // Tag masks E_K(J0): formed in row 0's keystream pass when that row has
    // ciphertext lanes (the segment that starts a record adds it); otherwise
    // here, for the record whose last row ends segment s, by lane 0 of wave s
    // before its rows (one lane per wave: the view is read as a scalar).
    {
        const uint32_t s = tid >> 6;
        if (!sch.ek_row0 && (tid & 63u) == 0 && s < nseg && (s ? qb1 : qb0) == sch.rows) {
            const RecView v = get_view(s_view + 5 * s);
            uint32_t ek[4];
            aes_ctr_block(aes, aes_lane(0), keys, bswap32(v.iv[0]) ^ ctx->rk[0], bswap32(v.iv[1]) ^ ctx->rk[1],
                          bswap32(v.iv[2]) ^ ctx->rk[2], 1u, ek);
            s_ek[s] = make_uint4(ek[0], ek[1], ek[2], ek[3]);
        }
    }

    const AesLane lane = aes_lane(tid & 63u);
    uint4* const s_p0 = ptab0;  // two segments: segment 0's products during segment 1
    // Rows of segment s; the unit's partial, moved onto the segment's
    // exponent grid.  A straddling workgroup parks segment 0's in s_p0, a
    // pair (whose table holds that region) in global memory.
    auto segment = [&](const uint32_t s) __attribute__((always_inline)) -> uint4 {
        const uint32_t qa = s ? 0u : qa0, qb = s ? qb1 : qb0;
        const RecView v = get_view(s_view + 5 * s);
        uint32_t y[4];
        unit_rows<kMode, kAligned, kWT>(ctx, sch, v, g_u, g_u2, aes, lane, keys, t, u, qa, qb, s_ek + s, y);
        // d = segment rows after the unit's last row (0 when it has none).
        const uint32_t J = qb - qa;
        const uint32_t d = u < J ? (J - 1 - u) % SI_U : 0u;
        uint32_t pr[4];
        if (d == 1) gh_mul(g_1, y, pr);
        else if (d == 2) gh_mul(g_2, y, pr);
        else { pr[0] = y[0]; pr[1] = y[1]; pr[2] = y[2]; pr[3] = y[3]; }
        const uint4 r = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        if (s == 0 && nseg == 2) {
            if (pair) sch.park[uint64_t(blockIdx.x) * SI_NT + tid] = r;
            else s_p0[tid] = r;
        }
        return r;
    };
    uint4 p = segment(0);
    if (nseg == 2) p = segment(1);
    // A pair's segment-0 product back from global memory (this thread's own
    // store; the load overlaps the tag read and the barrier below).
    const uint4 p0 = pair ? sch.park[uint64_t(blockIdx.x) * SI_NT + tid] : make_uint4(0, 0, 0, 0);
    // The expected tag of each record, loaded now so that the read is off the
    // finalising workgroup's critical path (it is needed after the ticket).
    // Lanes 0 and 1 read different views, so the pointer stays per lane
    // (RecView::tag is bytes 24..31 of the view: word 1, .z/.w).
    uint4 tag_pre = make_uint4(0, 0, 0, 0);
    if (kMode != MODE_ENCRYPT && tid < nseg) {
        static_assert(offsetof(RecView, tag) == 24, "view word 1, high half");
        const uint4 w1 = s_view[5 * tid + 1];
        const uint8_t* tp = reinterpret_cast<const uint8_t*>(uint64_t(w1.z) | (uint64_t(w1.w) << 32));
        if ((reinterpret_cast<uintptr_t>(tp) & 15u) == 0) {
            tag_pre = gload4(tp);
        } else {
            uint32_t w4[4];
            load_block<false>(tp, 16u, w4);
            tag_pre = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    }
    __syncthreads();  // AES and GHASH tables are dead from here on

    // The last segment's products to LDS; placement t is shared by the three
    // threads (u, t): one table, three nibble classes.
    xs[u * SI_T + t] = p;
    if (pair) xs0[u * SI_T + t] = p0;
    __syncthreads();
    uint32_t w[2][4];
    unit_sum(xs, t, w[1]);
    uint32_t q[2][4];
    if (nseg == 1) {  // uniform over the workgroup; the table is ready
        const uint32_t(&x1)[1][4] = reinterpret_cast<const uint32_t(&)[1][4]>(w[1]);
        uint32_t(&o1)[1][4] = reinterpret_cast<uint32_t(&)[1][4]>(q[1]);
        const uint4* const tb[1] = {ptab0};
        place_part<1>(u, x1, tb, s_zero, t, o1);
    } else {
        const uint4* const s_w0 = pair ? xs0 : s_p0;
        unit_sum(s_w0, t, w[0]);
        if (!pair) {  // uniform over the workgroup
            const uint4 z0 = s_zp[t], z1 = s_zp[SI_T + t];
            __syncthreads();  // s_p0 and s_zp are read; the region takes segment 0's table
            {
                const uint32_t za[4] = {z0.x, z0.y, z0.z, z0.w}, zb[4] = {z1.x, z1.y, z1.z, z1.w};
                gh_table_share<SI_U>(za, u, ptab0, t, SI_T);
                gh_table_share<SI_U>(zb, u, ptab1, t, SI_T);
            }
            __syncthreads();
        }
        const uint4* const tb[2] = {ptab0, pair ? ptab0 : ptab1};
        place_part<2>(u, w, tb, s_zero, t, q);
        wave_xor4_to63(q[0]);
        if ((tid & 63u) == 63u) s_c0[tid >> 6] = make_uint4(q[0][0], q[0][1], q[0][2], q[0][3]);
    }
    wave_xor4_to63(q[1]);
    if ((tid & 63u) == 63u) s_red[tid >> 6] = make_uint4(q[1][0], q[1][1], q[1][2], q[1][3]);
    // Every wave's data stores must be complete (write-through) or at least
    // in L2 (before the ticket's release) when the ticket is taken;
    // s_barrier does not wait for them.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid < nseg) {
        const uint32_t s = tid;
        const uint32_t qa = s ? 0u : qa0, qb = s ? qb1 : qb0;
        uint32_t r4[4] = {0, 0, 0, 0};
        const uint4* red = (s == 0 && nseg == 2) ? s_c0 : s_red;
#pragma unroll
        for (int w = 0; w < SI_NT / 64; ++w) {
            const uint4 e = red[w];
            r4[0] ^= e.x; r4[1] ^= e.y; r4[2] ^= e.z; r4[3] ^= e.w;
        }
        if (sch.ek_row0 ? qa == 0 : qb == sch.rows) {  // the record's tag mask
            const uint4 e = s_ek[s];
            r4[0] ^= e.x; r4[1] ^= e.y; r4[2] ^= e.z; r4[3] ^= e.w;
        }
        if (qb == sch.rows) {  // the length block's term
            r4[0] ^= sch.lh[0]; r4[1] ^= sch.lh[1]; r4[2] ^= sch.lh[2]; r4[3] ^= sch.lh[3];
        }
        uint32_t last = 1;
        if (qa != 0 || qb != sch.rows) {
            RecAcc* ra = acc + r0 + s;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                __hip_atomic_fetch_xor(&ra->w[k], r4[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // Count this segment's rows once its data stores and XORs are
            // performed.  Write-through stores are complete after s_waitcnt;
            // byte-granular stores need the agent-scope release (L2 write-back).
            uint32_t prev;
            if (kNeedRelease) {
                prev = __hip_atomic_fetch_add(&ra->count, qb - qa, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __builtin_amdgcn_s_waitcnt(0);
                prev = __hip_atomic_fetch_add(&ra->count, qb - qa, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            last = prev + (qb - qa) == sch.rows ? 1u : 0u;
            if (last) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    r4[k] = __hip_atomic_exchange(&ra->w[k], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&ra->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        s_last[s] = last;
        s_fin[s][0] = r4[0]; s_fin[s][1] = r4[1]; s_fin[s][2] = r4[2]; s_fin[s][3] = r4[3];
        s_tag[s] = tag_pre;
    }
    __syncthreads();

    // Finalise the records completed here.
#pragma unroll 1
    for (uint32_t s = 0; s < nseg; ++s) {
        if (!s_last[s]) continue;
        const RecView v = get_view(s_view + 5 * s);
        if (kMode == MODE_ENCRYPT) {
            // A record whose block-table entry is out of range gets the
            // complement of its tag, which never verifies: the host rejects
            // it whether or not the caller reads the fail counter.
            if (tid == 0 && v.bad && v.fail_count) atomicAdd(v.fail_count, 1u);
            if (tid < 4) {
                const uint32_t w = s_fin[s][tid] ^ (v.bad ? 0xffffffffu : 0u);
                for (int b = 0; b < 4; ++b) gmem(v.tag)[4 * tid + b] = uint8_t(w >> (8 * b));
            }
            continue;
        }
        const uint4 et = s_tag[s];
        const uint32_t diff = (s_fin[s][0] ^ et.x) | (s_fin[s][1] ^ et.y) | (s_fin[s][2] ^ et.z) | (s_fin[s][3] ^ et.w);
        const uint32_t ok = (diff == 0 && !v.bad) ? 1u : 0u;
        if (tid == 0) {
            *gmem(v.status) = ok;
            if (sch.status_out) gmem(sch.status_out)[r0 + s] = ok;
            if (!ok && v.fail_count) atomicAdd(v.fail_count, 1u);
        }
        if (!ok && kMode != MODE_VERIFY && !v.skip) zero_bytes(v.dst, sch.bytes, tid, SI_NT);
    }
}

template <int kMode, bool kAligned, bool kWT>
__global__ __launch_bounds__(SI_NT) __attribute__((amdgpu_waves_per_eu(SI_U, SI_U)))
void gcm_records_kernel(const GcmCtx* __restrict__ ctx, RecBatch batch, Sched sch,
                        RecAcc* __restrict__ acc)
{
    clock_stamp(sch.clock, 0);
    gcm_records_body<kMode, kAligned, kWT>(ctx, batch, sch, acc);
    clock_stamp(sch.clock, 1);
}

// Verify-before-release, second launch: record r (grid y) was verified by a
// MODE_VERIFY launch that wrote its status word; workgroup x decrypts blocks
// [x*chunk, (x+1)*chunk) of it into its destination (slot, or the codec
// staging row) only if that status is 1, and writes zeros there otherwise:
// the reference's order, tag first, then masked output
// (ghash.aicpu:623-648), so no unverified byte reaches the destination.
// A slot id out of range with no staging touches nothing.  A thread's
// blocks lie SI_RELEASE_THREADS apart, a multiple of 256, so its counter's
// low byte never changes, and the counter-mode cache of rounds 1-2 applies
// while counter bytes 12..13 stay fixed over the workgroup's range.
__device__ __forceinline__ void release_body(const GcmCtx* __restrict__ ctx, const RecBatch& b, uint64_t bytes,
                                             uint32_t chunk, int aligned, const uint32_t* gate)
{
    __shared__ uint32_t s_aes[256 * 64];
    if (gate && *gmem(gate) == 0u) return;
    const uint32_t tid = threadIdx.x, r = blockIdx.y;
    const RecView v = view_of(b, r);
    if (v.skip) return;
    const uint64_t nb = (bytes + 15) / 16;
    const uint64_t k0 = uint64_t(blockIdx.x) * chunk;
    if (k0 >= nb) return;
    const uint64_t k1 = k0 + chunk < nb ? k0 + chunk : nb;
    const uint32_t ok = (*gmem(v.status) == 1u && !v.bad) ? 1u : 0u;
    if (!ok) {
        const uint64_t e = 16 * k1 < bytes ? 16 * k1 : bytes;
        zero_bytes(v.dst + 16 * k0, e - 16 * k0, tid, SI_RELEASE_THREADS);
        return;
    }
    if (tid < 256) aes_fill_lds(s_aes, ctx->te0, tid);
    AesKeys keys;
    load_keys(ctx, keys);
    __syncthreads();
    const AesLane lane = aes_lane(tid & 63u);
    const uint32_t n0 = bswap32(v.iv[0]) ^ ctx->rk[0];
    const uint32_t n1 = bswap32(v.iv[1]) ^ ctx->rk[1];
    const uint32_t n2 = bswap32(v.iv[2]) ^ ctx->rk[2];
    const uint32_t clo = v.iv[3] + uint32_t(k0), chi = v.iv[3] + uint32_t(k1 - 1);
    const bool cached = chi >= clo && (clo >> 16) == (chi >> 16);  // uniform over the workgroup
    const bool fast = aligned && (bytes & 15) == 0;
    CtrCache cc{};
    if (cached) cc = ctr_cache(s_aes, lane, ctx, n0, n1, n2, bswap32(v.iv[3] + uint32_t(k0 + tid)) ^ keys.rk3);
    for (uint64_t k = k0 + tid; k < k1; k += SI_RELEASE_THREADS) {
        uint32_t ks[4];
        if (cached) aes_ctr_block_cached(s_aes, lane, keys, cc, v.iv[3] + uint32_t(k), ks);
        else aes_ctr_block(s_aes, lane, keys, n0, n1, n2, v.iv[3] + uint32_t(k), ks);
        if (fast) {
            const uint4 c = gload4(v.src + 16 * k);
            gstore4(v.dst + 16 * k, make_uint4(c.x ^ ks[0], c.y ^ ks[1], c.z ^ ks[2], c.w ^ ks[3]));
        } else {
            const uint32_t valid = k == nb - 1 ? uint32_t(bytes - 16 * k) : 16u;
            uint32_t c[4];
            load_block<true>(v.src + 16 * k, valid, c);  // wire records are 16-byte aligned
            const uint32_t o[4] = {c[0] ^ ks[0], c[1] ^ ks[1], c[2] ^ ks[2], c[3] ^ ks[3]};
            if (aligned) store_block<true>(v.dst + 16 * k, valid, o);
            else store_block<false>(v.dst + 16 * k, valid, o);
        }
    }
}

__global__ __launch_bounds__(SI_RELEASE_THREADS) void release_kernel(const GcmCtx* __restrict__ ctx, RecBatch b,
                                                                     uint64_t bytes, uint32_t chunk, int aligned,
                                                                     const uint32_t* gate, uint64_t* clock)
{
    clock_stamp(clock, 0);
    release_body(ctx, b, bytes, chunk, aligned, gate);
    clock_stamp(clock, 1);
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

// GHASH of aad || input || lengths by one workgroup: rows of SI_T blocks
// counted from the end (thread t owns block t of each row, Horner with the
// H^T tables in LDS), then thread t's sum times H^(T + 1 - t) from the power
// table, XORed over the workgroup with the length block's L * H.
__global__ __launch_bounds__(SI_T) void ghash_kernel(const GcmCtx* __restrict__ ctx, GhashJob j)
{
    __shared__ uint4 tbl[32 * 16];
    __shared__ uint4 wsum[SI_T / 64];
    __shared__ uint32_t s_ok;
    const uint32_t t = threadIdx.x;
    tbl[t] = ctx->gh4[t];
    tbl[SI_T + t] = ctx->gh4[SI_T + t];
    __syncthreads();
    const uint64_t a = (j.aad_bytes + 15) / 16, n = (j.input_bytes + 15) / 16, m = a + n;
    const uint64_t rows = (m + SI_T - 1) / SI_T;
    uint32_t y[4] = {0, 0, 0, 0};
    for (uint64_t q = 0; q < rows; ++q) {
        if (q) gh_mul_table(tbl, y);
        const int64_t i = int64_t(m) - int64_t(rows - q) * SI_T + int64_t(t);
        if (i < 0) continue;
        uint32_t x[4];
        if (uint64_t(i) < a) {
            const uint64_t off = uint64_t(i) * 16;
            load_block<false>(j.aad + off, uint32_t(j.aad_bytes - off < 16 ? j.aad_bytes - off : 16), x);
        } else {
            const uint64_t off = (uint64_t(i) - a) * 16;
            load_block<false>(j.input + off, uint32_t(j.input_bytes - off < 16 ? j.input_bytes - off : 16), x);
        }
        y[0] ^= x[0]; y[1] ^= x[1]; y[2] ^= x[2]; y[3] ^= x[3];
    }
    const uint4 pw = reinterpret_cast<const uint4*>(ctx + 1)[SI_T + 1 - t];
    const uint4 z = gf_mul4(make_uint4(y[0], y[1], y[2], y[3]), pw);
    uint32_t v[4] = {z.x, z.y, z.z, z.w};
    wave_xor4_to63(v);
    if ((t & 63u) == 63u) wsum[t >> 6] = make_uint4(v[0], v[1], v[2], v[3]);
    __syncthreads();
    if (t == 0) {
        uint32_t g[4] = {0, 0, 0, 0};
        for (uint32_t w = 0; w < SI_T / 64; ++w) {
            g[0] ^= wsum[w].x; g[1] ^= wsum[w].y; g[2] ^= wsum[w].z; g[3] ^= wsum[w].w;
        }
        // L = [bits(aad)]_64 || [bits(input)]_64, big-endian, as memory-order words.
        const uint64_t la = j.aad_bytes * 8, lc = j.input_bytes * 8;
        const uint4 L = make_uint4(bswap32(uint32_t(la >> 32)), bswap32(uint32_t(la)), bswap32(uint32_t(lc >> 32)),
                                   bswap32(uint32_t(lc)));
        const uint4 lh = gf_mul4(L, make_uint4(ctx->h[0], ctx->h[1], ctx->h[2], ctx->h[3]));
        g[0] ^= lh.x; g[1] ^= lh.y; g[2] ^= lh.z; g[3] ^= lh.w;
        if (j.flags & SI_GHASH_FINALIZE_TAG) {
            uint32_t mk[4];
            load_block<false>(j.tag_mask, 16u, mk);
            g[0] ^= mk[0]; g[1] ^= mk[1]; g[2] ^= mk[2]; g[3] ^= mk[3];
        }
        store_block<false>(j.output, 16u, g);
        uint32_t ok = 1;
        if (j.flags & SI_GHASH_VERIFY_TAG) {
            uint32_t e[4];
            load_block<false>(j.expected_tag, 16u, e);
            ok = ((g[0] ^ e[0]) | (g[1] ^ e[1]) | (g[2] ^ e[2]) | (g[3] ^ e[3])) == 0 ? 1u : 0u;
        }
        s_ok = ok;
    }
    __syncthreads();
    const uint32_t ok = s_ok;
    if (j.flags & SI_GHASH_XOR_ON_SUCCESS) {
        const uint32_t mask = 0u - ok;
        for (uint64_t k = t; k < n; k += SI_T) {
            const uint32_t valid = uint32_t(j.input_bytes - k * 16 < 16 ? j.input_bytes - k * 16 : 16);
            uint32_t c[4], ks[4];
            load_block<false>(j.input + 16 * k, valid, c);
            load_block<false>(j.keystream + 16 * k, valid, ks);
            const uint32_t o[4] = {(c[0] ^ ks[0]) & mask, (c[1] ^ ks[1]) & mask, (c[2] ^ ks[2]) & mask,
                                   (c[3] ^ ks[3]) & mask};
            store_block<false>(j.plaintext + 16 * k, valid, o);
        }
    }
    if (t == 0 && j.status) *gmem(j.status) = ok;
}

__global__ void auth_gate_kernel(uint8_t* data, const uint32_t* status, uint64_t bytes)
{
    if (*status == 1u) return;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride)
        data[i] = 0;
}

__global__ void zero_words_kernel(uint4* p, uint64_t n)
{
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

uint8_t* noalloc_scratch(hipStream_t stream)
{
    static std::mutex m;
    static std::map<int, uint8_t*> ptrs;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> g(m);
    auto it = ptrs.find(dev);
    if (it != ptrs.end()) return it->second;
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    // The owner word and the record kernel's accumulators must start at zero
    // (the workgroup that finalises a record returns its accumulator to
    // zero, and a finishing kernel returns the owner word to zero).  The
    // array is zero when the code object loads; this clear runs once per
    // device, before any call can hold the scratch (the lock is held until
    // it completes).  Under capture it is skipped: a clear recorded into a
    // graph would run again at every replay, under other calls' feet.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return nullptr;
    if (cs == hipStreamCaptureStatusNone) {
        const uint64_t words = (SI_NOALLOC_CTRL_BYTES + SI_NOALLOC_ACC_BYTES) / 16u;
        hipLaunchKernelGGL(zero_words_kernel, dim3(uint32_t((words + 255) / 256)), dim3(256), 0, stream,
                           static_cast<uint4*>(ptr), words);
        if (hipGetLastError() != hipSuccess) return nullptr;
        if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
    }
    ptrs[dev] = static_cast<uint8_t*>(ptr);
    return ptrs[dev];
}

// Control word 0: the owner token; word 1: the token sequence.
__global__ void noalloc_acquire_kernel(uint32_t* ctrl, uint32_t* cell)
{
    uint32_t tok;
    do {
        tok = __hip_atomic_fetch_add(&ctrl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    } while (tok == 0u || tok == SI_NOALLOC_TEST_TOKEN);
    uint32_t expected = 0u;
    const bool won = __hip_atomic_compare_exchange_strong(&ctrl[0], &expected, tok, __ATOMIC_ACQ_REL,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *gmem(cell) = won ? tok : 0u;
}

// One workgroup per record (grid nrec): release the owner word, or fail the
// denied call's records closed.
__global__ __launch_bounds__(256) void noalloc_finish_kernel(NoallocFinish f)
{
    const uint32_t tok = *gmem(f.cell);
    const uint32_t r = blockIdx.x;
    if (tok != 0u) {
        if (r == 0 && threadIdx.x == 0) {
            uint32_t expected = tok;
            __hip_atomic_compare_exchange_strong(&f.ctrl[0], &expected, 0u, __ATOMIC_ACQ_REL, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    if (threadIdx.x == 0) {
        *gmem(reinterpret_cast<uint32_t*>(f.wire + uint64_t(r) * f.wire_stride + f.status_off)) = 0u;
        if (f.status_out) gmem(f.status_out)[r] = 0u;
        if (r == 0 && f.fail_count) atomicAdd(f.fail_count, f.nrec);
    }
    const int64_t sid = f.slots[r];
    if (sid < 0 || sid >= f.nslots) return;  // a bad slot id touches no cache memory
    uint8_t* dst = f.cache[r < f.n_k ? 0 : 1] + uint64_t(sid) * f.slot_bytes;
    zero_bytes(dst, f.out_bytes, threadIdx.x, blockDim.x);
}

__global__ void noalloc_test_hold_kernel(uint32_t* ctrl, int hold)
{
    uint32_t expected = hold ? 0u : SI_NOALLOC_TEST_TOKEN;
    __hip_atomic_compare_exchange_strong(&ctrl[0], &expected, hold ? SI_NOALLOC_TEST_TOKEN : 0u, __ATOMIC_ACQ_REL,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

hipError_t launch_noalloc_acquire(hipStream_t stream, uint32_t* ctrl, uint32_t* cell)
{
    hipLaunchKernelGGL(noalloc_acquire_kernel, dim3(1), dim3(1), 0, stream, ctrl, cell);
    return hipGetLastError();
}

hipError_t launch_noalloc_finish(hipStream_t stream, const NoallocFinish& f)
{
    if (f.nrec == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(noalloc_finish_kernel, dim3(f.nrec), dim3(256), 0, stream, f);
    return hipGetLastError();
}

hipError_t launch_noalloc_test_hold(hipStream_t stream, uint32_t* ctrl, int hold)
{
    hipLaunchKernelGGL(noalloc_test_hold_kernel, dim3(1), dim3(1), 0, stream, ctrl, hold);
    return hipGetLastError();
}

// ---------------------------------------------------------------- launches

template <int kMode, bool kAligned, bool kWT>
static void launch_records(dim3 grid, dim3 block, hipStream_t stream, const LaunchEvents& ev, const GcmCtx* ctx,
                           const RecBatch& b, const Sched& s, RecAcc* acc)
{
    if (ev.start || ev.stop)
        hipExtLaunchKernelGGL((gcm_records_kernel<kMode, kAligned, kWT>), grid, block, 0, stream, ev.start, ev.stop,
                              0, ctx, b, s, acc);
    else
        hipLaunchKernelGGL((gcm_records_kernel<kMode, kAligned, kWT>), grid, block, 0, stream, ctx, b, s, acc);
}

template <int kMode>
static hipError_t launch_mode(hipStream_t stream, const GcmCtx* ctx, const RecBatch& b,
                              const Sched& s, RecAcc* acc, bool aligned, const LaunchEvents& ev)
{
    if (s.nwg == 0) return hipSuccess;
    const dim3 grid(s.nwg), block(SI_NT);
    if (ev.clock) {
        // a measured launch: the same schedule with this kernel's stamps
        Sched sm = s;
        sm.clock = ev.clock->take(uint64_t(s.nwg) * (SI_NT / 64));
        LaunchEvents e2 = ev;
        e2.clock = nullptr;
        return launch_mode<kMode>(stream, ctx, b, sm, acc, aligned, e2);
    }
    if (aligned && s.bytes % 16 == 0)
        launch_records<kMode, true, true>(grid, block, stream, ev, ctx, b, s, acc);
    else if (aligned)
        launch_records<kMode, true, false>(grid, block, stream, ev, ctx, b, s, acc);
    else
        launch_records<kMode, false, false>(grid, block, stream, ev, ctx, b, s, acc);
    return hipGetLastError();
}

hipError_t launch_gcm(int mode, hipStream_t stream, const GcmCtx* ctx, const RecBatch& b,
                      const Sched& s, RecAcc* acc, bool aligned, const LaunchEvents& ev)
{
    switch (mode) {
    case MODE_DECRYPT: return launch_mode<MODE_DECRYPT>(stream, ctx, b, s, acc, aligned, ev);
    case MODE_ENCRYPT: return launch_mode<MODE_ENCRYPT>(stream, ctx, b, s, acc, aligned, ev);
    case MODE_VERIFY: return launch_mode<MODE_VERIFY>(stream, ctx, b, s, acc, aligned, ev);
    case MODE_VERIFY_XOR: return launch_mode<MODE_VERIFY_XOR>(stream, ctx, b, s, acc, aligned, ev);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_release(hipStream_t stream, const GcmCtx* ctx, const RecBatch& b, uint32_t nrec, uint64_t bytes,
                          bool aligned, const uint32_t* gate, uint32_t cus, const LaunchEvents& ev)
{
    if (nrec == 0) return hipSuccess;
    // Blocks per workgroup: the grid fills each CU's two workgroup slots (64
    // KiB of LDS each) once, k = 2 * cus / nrec workgroups per record, in
    // multiples of 256 blocks.  Against a fixed 4,096 blocks per workgroup
    // (MI355X, verify-before-release layers, ABBA on one GPU): bf16
    // Llama-3-8B 50.9 -> 47.1 us, int4 Qwen2.5-7B 33.4 -> 29.6, int8
    // Llama-3-8B 57.5 -> 50.8 (the int4 layer's 128 records had filled only
    // half the CUs).
    const uint64_t nb = (bytes + 15) / 16;
    const uint64_t per = cus && 2ull * cus > nrec ? 2ull * cus / nrec : 1ull;
    uint64_t chunk = (nb + per - 1) / per;
    chunk = (chunk + 255) / 256 * 256;
    const dim3 grid(uint32_t((nb + chunk - 1) / chunk), nrec), block(SI_RELEASE_THREADS);
    uint64_t* clock = ev.clock ? ev.clock->take(uint64_t(grid.x) * grid.y * (SI_RELEASE_THREADS / 64)) : nullptr;
    if (ev.start || ev.stop)
        hipExtLaunchKernelGGL(release_kernel, grid, block, 0, stream, ev.start, ev.stop, 0, ctx, b, bytes,
                              uint32_t(chunk), aligned ? 1 : 0, gate, clock);
    else
        hipLaunchKernelGGL(release_kernel, grid, block, 0, stream, ctx, b, bytes, uint32_t(chunk), aligned ? 1 : 0,
                           gate, clock);
    return hipGetLastError();
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

hipError_t launch_ghash(hipStream_t stream, const GcmCtx* ctx, const GhashJob& j)
{
    hipLaunchKernelGGL(ghash_kernel, dim3(1), dim3(SI_T), 0, stream, ctx, j);
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
