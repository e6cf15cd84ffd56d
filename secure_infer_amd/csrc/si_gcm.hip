// AES-128-GCM record kernels for gfx950.
//
// One launch processes a batch of records.  Each record's GHASH input is the
// block sequence X = AAD || C || L (SP 800-38D), m = a + n + 1 blocks, and
// GHASH = XOR_k X_k * H^(m-k).  The record is cut into NC chunks of CH = J*T
// blocks, counted from the end of X; workgroup (r, c) owns chunk c and thread
// t of it owns blocks base_c + j*T + t (j = 0..J-1), so every row of a chunk
// is one coalesced 4 KiB sweep.  Per thread:
//   * CTR: keystream of counter iv3 + k for ciphertext block k (32-bit wrap,
//     ghash.aicpu:174-221), XORed into the data and stored;
//   * GHASH: Horner with H^T over the thread's blocks (LDS tables), then one
//     generic multiply by H^(c*CH + T - t) from the per-key power table, which
//     places the thread's partial at its true exponent.
// Partials are XOR-reduced over the workgroup and then across workgroups with
// device-scope atomics; the last workgroup of a record (atomic ticket) adds
// nothing more, compares the tag in constant time, writes the status and, on
// failure, zeroes the record's output before the kernel ends.  Every
// workgroup publishes its stores with an agent-scope release before taking
// the ticket, so the zeroing is ordered after all plaintext stores.
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

template <int kMode, bool kAligned>
__global__ __launch_bounds__(SI_T) void gcm_records_kernel(const GcmCtx* __restrict__ ctx,
                                                           RecBatch batch, Sched sch,
                                                           RecAcc* __restrict__ acc)
{
    __shared__ uint32_t s_aes[256 * 64];  // AES tables; reused for the generic multiply
    __shared__ uint4 s_gh[32 * 16];
    __shared__ uint32_t s_red[SI_T / 64][4];
    __shared__ uint32_t s_last;

    const uint32_t tid = threadIdx.x;
    aes_fill_lds(s_aes, ctx->te0, tid, SI_T);
    for (uint32_t i = tid; i < 32u * 16u; i += SI_T) s_gh[i] = ctx->gh4[i];
    __syncthreads();

    const uint32_t r = blockIdx.x / sch.nc;
    const uint32_t c = blockIdx.x % sch.nc;
    const RecView v = view_of(batch, r);
    const AesLane lane = aes_lane(tid & 63u);
    const uint32_t n0 = bswap32(v.iv[0]) ^ ctx->rk[0];
    const uint32_t n1 = bswap32(v.iv[1]) ^ ctx->rk[1];
    const uint32_t n2 = bswap32(v.iv[2]) ^ ctx->rk[2];

    const int64_t m = int64_t(sch.a) + int64_t(sch.n) + 1;
    const int64_t ch = int64_t(sch.j) * SI_T;
    const int64_t base = m - int64_t(c + 1) * ch;
    const uint32_t tail = uint32_t(sch.bytes - (uint64_t(sch.n) - 1) * 16u);  // bytes in last block
    const uint32_t aad_tail = sch.aad_bytes ? uint32_t(sch.aad_bytes - (uint64_t(sch.a) - 1) * 16u) : 0u;

    uint32_t y[4] = {0, 0, 0, 0};
    for (uint32_t j = 0; j < sch.j; ++j) {
        if (j != 0) gh_mul_table(s_gh, y);
        const int64_t i = base + int64_t(j) * SI_T + tid;
        if (i < 0) continue;
        uint32_t x[4];
        if (i >= int64_t(sch.a) && i < int64_t(sch.a) + int64_t(sch.n)) {
            if (v.bad && !batch.staging) continue;
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
                    aes_ctr_block(s_aes, lane, ctx, n0, n1, n2, v.iv[3] + uint32_t(k), ks);
                }
                uint32_t out[4] = {in[0] ^ ks[0], in[1] ^ ks[1], in[2] ^ ks[2], in[3] ^ ks[3]};
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

    // Tag mask E_K(J0), J0 = nonce || 1, folded in by the owner of block m-1.
    uint32_t ek[4] = {0, 0, 0, 0};
    const bool owns_len = c == 0 && tid == SI_T - 1;
    if (owns_len) aes_ctr_block(s_aes, lane, ctx, n0, n1, n2, 1u, ek);
    __syncthreads();  // AES tables are dead from here on

    const int64_t i_last = base + int64_t(sch.j - 1) * SI_T + tid;
    uint32_t q[4] = {0, 0, 0, 0};
    {
        const uint64_t e = i_last >= 0 ? uint64_t(c) * uint64_t(ch) + SI_T - tid : 0u;
        const uint4 zp = reinterpret_cast<const uint4*>(ctx + 1)[e];
        const uint32_t z[4] = {zp.x, zp.y, zp.z, zp.w};
        gh_mul_generic(y, z, reinterpret_cast<uint4*>(s_aes), tid, SI_T, q);
    }
    q[0] ^= ek[0]; q[1] ^= ek[1]; q[2] ^= ek[2]; q[3] ^= ek[3];
    wave_xor4(q);
    // Every wave's data stores must have reached L2 before thread 0's
    // agent-scope release below writes L2 back (s_barrier does not wait).
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
        if (sch.nc == 1) {
            s_red[0][0] = t[0]; s_red[0][1] = t[1]; s_red[0][2] = t[2]; s_red[0][3] = t[3];
            s_last = 1;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                __hip_atomic_fetch_xor(&ra->w[k], t[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // Release this workgroup's data stores and XORs, take a ticket.
            const uint32_t prev = __hip_atomic_fetch_add(&ra->count, 1u, __ATOMIC_ACQ_REL,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            s_last = prev == sch.nc - 1 ? 1u : 0u;
            if (s_last) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    s_red[0][k] = __hip_atomic_exchange(&ra->w[k], 0u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&ra->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    __syncthreads();
    if (!s_last) return;

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

// ---------------------------------------------------------------- CTR only

__global__ __launch_bounds__(SI_T) void ctr_kernel(const GcmCtx* __restrict__ ctx,
                                                   const uint8_t* __restrict__ in,
                                                   uint8_t* __restrict__ out, uint64_t bytes,
                                                   uint4 iv, int aligned)
{
    __shared__ uint32_t s_aes[256 * 64];
    const uint32_t tid = threadIdx.x;
    aes_fill_lds(s_aes, ctx->te0, tid, SI_T);
    __syncthreads();
    const AesLane lane = aes_lane(tid & 63u);
    const uint32_t n0 = bswap32(iv.x) ^ ctx->rk[0];
    const uint32_t n1 = bswap32(iv.y) ^ ctx->rk[1];
    const uint32_t n2 = bswap32(iv.z) ^ ctx->rk[2];
    const uint64_t nb = (bytes + 15) / 16;
    for (uint64_t k = uint64_t(blockIdx.x) * SI_T + tid; k < nb; k += uint64_t(gridDim.x) * SI_T) {
        const uint32_t valid = k == nb - 1 ? uint32_t(bytes - 16 * k) : 16u;
        uint32_t ks[4], d[4] = {0, 0, 0, 0};
        aes_ctr_block(s_aes, lane, ctx, n0, n1, n2, iv.w + uint32_t(k), ks);
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
    const dim3 grid(s.nc * s.nrec), block(SI_T);
    if (aligned)
        hipLaunchKernelGGL((gcm_records_kernel<kMode, true>), grid, block, 0, stream, ctx, b, s, acc);
    else
        hipLaunchKernelGGL((gcm_records_kernel<kMode, false>), grid, block, 0, stream, ctx, b, s, acc);
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
