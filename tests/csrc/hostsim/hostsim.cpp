// TEST INFRASTRUCTURE ONLY: the host-only stand-in for the HIP runtime and
// for the library's kernels that lets the library's host code (si_api.cpp,
// si_host.cpp) run on the CPU under ThreadSanitizer and AddressSanitizer.
//
//  * A stream is a worker thread that runs its tasks in order; an event is a
//    generation counter that a stream task completes; a stream wait is a task
//    that blocks until the event's generation at the time of the call has
//    completed.  Every hand-over between threads goes through a mutex, so the
//    sanitizers see exactly the orderings HIP guarantees and nothing more.
//  * Device memory is host memory (mapped pinned memory is the same pointer).
//  * The layer kernels the host code launches run as CPU tasks on their
//    stream with the same effects on the same buffers: AES-128-GCM with
//    OpenSSL (open / seal a record, status word, zeroed output, fail count),
//    the verify-before-release second launch (AES-CTR), the transport codec
//    through the oracle's C restatement, and the allocation-free entry's
//    scratch ownership.  Kernels the host runtime never launches (agreement,
//    kernel-level mirrors) report an error.
// Nothing here is linked into the product library.
#include <hip/hip_runtime.h>
#include <openssl/evp.h>

#include <array>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "si_kernels.h"
#include "si_layout.h"
#include "si_oracle.h"

// ---------------------------------------------------------------- streams

struct ihipStream_t {
    std::mutex m;
    std::condition_variable cv;
    std::deque<std::function<void()>> q;
    uint64_t queued = 0, done = 0;
    bool stop = false;
    std::thread th;

    ihipStream_t() : th([this] { run(); }) {}
    ~ihipStream_t()
    {
        {
            std::lock_guard<std::mutex> g(m);
            stop = true;
        }
        cv.notify_all();
        th.join();
    }
    void run()
    {
        for (;;) {
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> g(m);
                cv.wait(g, [&] { return stop || !q.empty(); });
                if (q.empty()) return;
                f = std::move(q.front());
                q.pop_front();
            }
            f();
            {
                std::lock_guard<std::mutex> g(m);
                ++done;
            }
            cv.notify_all();
        }
    }
    void push(std::function<void()> f)
    {
        {
            std::lock_guard<std::mutex> g(m);
            q.push_back(std::move(f));
            ++queued;
        }
        cv.notify_all();
    }
    void sync()
    {
        std::unique_lock<std::mutex> g(m);
        const uint64_t target = queued;
        cv.wait(g, [&] { return done >= target; });
    }
};

namespace {

// Live streams, shared: a hipDeviceSynchronize on one thread may still be
// syncing a stream that another thread is destroying (HIP allows both), so
// the object goes when its last holder lets go.
std::mutex g_streams_m;
std::map<ihipStream_t*, std::shared_ptr<ihipStream_t>>& g_streams =
    *new std::map<ihipStream_t*, std::shared_ptr<ihipStream_t>>();

ihipStream_t* new_stream()
{
    auto p = std::make_shared<ihipStream_t>();
    std::lock_guard<std::mutex> g(g_streams_m);
    g_streams[p.get()] = p;
    return p.get();
}

ihipStream_t* default_stream()
{
    static ihipStream_t* s = new_stream();
    return s;
}

ihipStream_t* S(hipStream_t s) { return s ? s : default_stream(); }

}  // namespace

// ---------------------------------------------------------------- events

struct ihipEvent_t {
    std::mutex m;
    std::condition_variable cv;
    uint64_t recorded = 0, completed = 0;
    std::chrono::steady_clock::time_point t{};
};

namespace {

// Handles map to shared objects, so a task still queued keeps its event alive
// after hipEventDestroy (HIP defers the release the same way).
std::mutex g_events_m;
std::map<ihipEvent_t*, std::shared_ptr<ihipEvent_t>>& g_events = *new std::map<ihipEvent_t*, std::shared_ptr<ihipEvent_t>>();

std::shared_ptr<ihipEvent_t> E(hipEvent_t e)
{
    std::lock_guard<std::mutex> g(g_events_m);
    auto it = g_events.find(e);
    if (it == g_events.end()) {
        fprintf(stderr, "[hostsim] use of an unknown or destroyed event %p\n", static_cast<void*>(e));
        abort();
    }
    return it->second;
}

}  // namespace

hipError_t hipGetDevice(int* dev)
{
    *dev = 0;
    return hipSuccess;
}

hipError_t hipSetDevice(int dev) { return dev == 0 ? hipSuccess : hipErrorInvalidValue; }

hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int)
{
    if (a == hipDeviceAttributeWallClockRate) {
        *v = 100000;  // kHz
        return hipSuccess;
    }
    if (a != hipDeviceAttributeMultiprocessorCount) return hipErrorInvalidValue;
    *v = 256;
    return hipSuccess;
}

hipError_t hipDeviceSynchronize(void)
{
    std::vector<std::shared_ptr<ihipStream_t>> all;
    {
        std::lock_guard<std::mutex> g(g_streams_m);
        for (auto& e : g_streams) all.push_back(e.second);
    }
    for (auto& s : all) s->sync();
    return hipSuccess;
}

hipError_t hipGetLastError(void) { return hipSuccess; }

hipError_t hipMalloc(void** p, size_t n)
{
    *p = aligned_alloc(256, (n + 255) / 256 * 256 + 256);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}

hipError_t hipFree(void* p)
{
    free(p);
    return hipSuccess;
}

hipError_t hipMallocAsync(void** p, size_t n, hipStream_t) { return hipMalloc(p, n); }

hipError_t hipFreeAsync(void* p, hipStream_t s)
{
    S(s)->push([p] { free(p); });
    return hipSuccess;
}

hipError_t hipHostMalloc(void** p, size_t n, unsigned int) { return hipMalloc(p, n); }

hipError_t hipHostFree(void* p) { return hipFree(p); }

hipError_t hipHostGetDevicePointer(void** dev, void* host, unsigned int)
{
    *dev = host;
    return hipSuccess;
}

hipError_t hipMemcpy(void* dst, const void* src, size_t n, hipMemcpyKind)
{
    memcpy(dst, src, n);
    return hipSuccess;
}

hipError_t hipMemset(void* p, int v, size_t n)
{
    memset(p, v, n);
    return hipSuccess;
}

hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t s)
{
    S(s)->push([=] { memcpy(dst, src, n); });
    return hipSuccess;
}

hipError_t hipMemcpy2DAsync(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                            hipMemcpyKind, hipStream_t s)
{
    S(s)->push([=] {
        for (size_t i = 0; i < height; ++i)
            memcpy(static_cast<uint8_t*>(dst) + i * dpitch, static_cast<const uint8_t*>(src) + i * spitch, width);
    });
    return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned int)
{
    *s = new_stream();
    return hipSuccess;
}

hipError_t hipStreamDestroy(hipStream_t s)
{
    if (!s) return hipErrorInvalidValue;
    std::shared_ptr<ihipStream_t> p;
    {
        std::lock_guard<std::mutex> g(g_streams_m);
        auto it = g_streams.find(s);
        if (it == g_streams.end()) return hipErrorInvalidValue;
        p = std::move(it->second);
        g_streams.erase(it);
    }
    p->sync();  // its queued work completes; the object goes with its last holder
    return hipSuccess;
}

hipError_t hipStreamSynchronize(hipStream_t s)
{
    S(s)->sync();
    return hipSuccess;
}

hipError_t hipEventCreate(hipEvent_t* e)
{
    auto p = std::make_shared<ihipEvent_t>();
    *e = p.get();
    std::lock_guard<std::mutex> g(g_events_m);
    g_events[p.get()] = p;
    return hipSuccess;
}

hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned int) { return hipEventCreate(e); }

hipError_t hipEventDestroy(hipEvent_t e)
{
    std::lock_guard<std::mutex> g(g_events_m);
    return g_events.erase(e) ? hipSuccess : hipErrorInvalidValue;
}

hipError_t hipEventRecord(hipEvent_t e, hipStream_t s)
{
    auto ev = E(e);
    uint64_t gen;
    {
        std::lock_guard<std::mutex> g(ev->m);
        gen = ++ev->recorded;
    }
    S(s)->push([ev, gen] {
        {
            std::lock_guard<std::mutex> g(ev->m);
            if (gen > ev->completed) {
                ev->completed = gen;
                ev->t = std::chrono::steady_clock::now();
            }
        }
        ev->cv.notify_all();
    });
    return hipSuccess;
}

hipError_t hipEventSynchronize(hipEvent_t e)
{
    auto ev = E(e);
    std::unique_lock<std::mutex> g(ev->m);
    const uint64_t gen = ev->recorded;
    ev->cv.wait(g, [&] { return ev->completed >= gen; });
    return hipSuccess;
}

hipError_t hipEventQuery(hipEvent_t e)
{
    auto ev = E(e);
    std::lock_guard<std::mutex> g(ev->m);
    return ev->completed >= ev->recorded ? hipSuccess : hipErrorNotReady;
}

hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b)
{
    auto ea = E(a), eb = E(b);
    std::chrono::steady_clock::time_point ta, tb;
    {
        std::lock_guard<std::mutex> g(ea->m);
        ta = ea->t;
    }
    {
        std::lock_guard<std::mutex> g(eb->m);
        tb = eb->t;
    }
    *ms = std::chrono::duration<float, std::milli>(tb - ta).count();
    return hipSuccess;
}

hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned int)
{
    auto ev = E(e);
    uint64_t gen;
    {
        std::lock_guard<std::mutex> g(ev->m);
        gen = ev->recorded;
    }
    S(s)->push([ev, gen] {
        std::unique_lock<std::mutex> g(ev->m);
        ev->cv.wait(g, [&] { return ev->completed >= gen; });
    });
    return hipSuccess;
}

// ---------------------------------------------------------------- kernels

namespace si {
namespace {

void key_of(const GcmCtx* ctx, uint8_t key[16])
{
    for (int i = 0; i < 4; ++i)
        for (int b = 0; b < 4; ++b) key[4 * i + b] = uint8_t(ctx->rk[i] >> (8 * b));
}

void put_be32(uint8_t* p, uint32_t v)
{
    p[0] = uint8_t(v >> 24);
    p[1] = uint8_t(v >> 16);
    p[2] = uint8_t(v >> 8);
    p[3] = uint8_t(v);
}

void add_u32(uint32_t* p, uint32_t v) { __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }

// Record r of a layer batch, as the device kernels see it.
struct View {
    const uint8_t* src;
    uint8_t* dst;
    const uint8_t* aad;
    uint8_t* tag;
    uint32_t* status;
    uint8_t iv12[12];
    bool bad, skip;
};

View view(const RecBatch& b, uint32_t r)
{
    View v{};
    uint8_t* wire = const_cast<uint8_t*>(b.wire) + uint64_t(r) * b.wire_stride;
    const uint32_t kind = r < b.n_k ? 0u : 1u;
    const int64_t sid = b.slots[r];
    v.bad = sid < 0 || sid >= b.nslots;
    v.skip = v.bad && !b.staging;
    uint8_t* slot = b.cache[kind] + uint64_t(v.bad ? 0 : sid) * b.slot_bytes;
    uint8_t* plain = b.staging ? b.staging + uint64_t(r) * b.staging_stride : slot;
    v.src = b.encrypt ? plain : wire;
    v.dst = b.encrypt ? wire : plain;
    v.aad = wire + b.aad_off;
    v.tag = wire + b.tag_off;
    v.status = reinterpret_cast<uint32_t*>(wire + b.status_off);
    uint32_t w[3];
    if (b.ivs) {
        w[0] = b.ivs[4 * r];
        w[1] = b.ivs[4 * r + 1];
        w[2] = b.ivs[4 * r + 2];
    } else {
        const uint64_t nonce = b.nonce_base + r;
        w[0] = b.iv[0];
        w[1] = uint32_t(nonce >> 32);
        w[2] = uint32_t(nonce);
    }
    for (int i = 0; i < 3; ++i) put_be32(v.iv12 + 4 * i, w[i]);
    return v;
}

bool gcm(bool enc, const uint8_t key[16], const uint8_t iv[12], const uint8_t* aad, const uint8_t* in, size_t n,
         uint8_t* out, uint8_t tag[16])
{
    EVP_CIPHER_CTX* c = EVP_CIPHER_CTX_new();
    int len = 0;
    bool ok = c && EVP_CipherInit_ex(c, EVP_aes_128_gcm(), nullptr, key, iv, enc ? 1 : 0) == 1 &&
              EVP_CipherUpdate(c, nullptr, &len, aad, 64) == 1 && EVP_CipherUpdate(c, out, &len, in, int(n)) == 1;
    if (ok && !enc) ok = EVP_CIPHER_CTX_ctrl(c, EVP_CTRL_GCM_SET_TAG, 16, tag) == 1;
    if (ok) ok = EVP_CipherFinal_ex(c, out + len, &len) == 1;
    if (ok && enc) ok = EVP_CIPHER_CTX_ctrl(c, EVP_CTRL_GCM_GET_TAG, 16, tag) == 1;
    EVP_CIPHER_CTX_free(c);
    return ok;
}

void ctr(const uint8_t key[16], const uint8_t iv12[12], const uint8_t* in, size_t n, uint8_t* out)
{
    uint8_t iv[16];
    memcpy(iv, iv12, 12);
    put_be32(iv + 12, 2);
    EVP_CIPHER_CTX* c = EVP_CIPHER_CTX_new();
    int len = 0;
    if (!c || EVP_EncryptInit_ex(c, EVP_aes_128_ctr(), nullptr, key, iv) != 1 ||
        EVP_EncryptUpdate(c, out, &len, in, int(n)) != 1 || EVP_EncryptFinal_ex(c, out + len, &len) != 1) {
        fprintf(stderr, "[hostsim] AES-CTR failed\n");
        abort();
    }
    EVP_CIPHER_CTX_free(c);
}

bool gated(const uint32_t* gate) { return gate && __atomic_load_n(gate, __ATOMIC_SEQ_CST) == 0u; }

// (layer, kind, block id, ticket) of every reload record, read from its AAD
// (secure_infer_build_gcm_aad: kind at byte 6, layer BE32 at 8, block id BE64
// at 12, ticket BE64 at 36), so the stress driver can check the order in
// which tickets were assigned.
std::mutex g_log_m;
std::vector<std::array<uint64_t, 4>>& g_log = *new std::vector<std::array<uint64_t, 4>>();

uint64_t be(const uint8_t* p, int n)
{
    uint64_t v = 0;
    for (int i = 0; i < n; ++i) v = (v << 8) | p[i];
    return v;
}

// Layer batches: 0 verify + decrypt (output zeroed on failure), 1 encrypt +
// tag (a bad slot id gets the complement of its tag), 2 verify only.
void layer_kernel(int mode, const GcmCtx* ctx, const RecBatch& b, const Sched& s)
{
    if (gated(s.gate)) return;
    uint8_t key[16];
    key_of(ctx, key);
    std::vector<uint8_t> tmp(s.bytes + 16), zero(s.bytes, 0);
    for (uint32_t r = 0; r < s.nrec; ++r) {
        const View v = view(b, r);
        if (mode == 1) {
            const uint8_t* pt = v.skip ? zero.data() : v.src;
            uint8_t* ct = v.skip ? tmp.data() : v.dst;
            if (!gcm(true, key, v.iv12, v.aad, pt, s.bytes, ct, v.tag)) abort();
            if (v.bad) {
                for (int i = 0; i < 16; ++i) v.tag[i] ^= 0xff;
                if (b.fail_count) add_u32(b.fail_count, 1);
            }
            continue;
        }
        {
            std::lock_guard<std::mutex> g(g_log_m);
            g_log.push_back({be(v.aad + 8, 4), v.aad[6], be(v.aad + 12, 8), be(v.aad + 36, 8)});
        }
        uint8_t tag[16];
        memcpy(tag, v.tag, 16);
        const uint32_t ok = (!v.bad && gcm(false, key, v.iv12, v.aad, v.src, s.bytes, tmp.data(), tag)) ? 1u : 0u;
        if (mode == 0 && !v.skip) memcpy(v.dst, ok ? tmp.data() : zero.data(), s.bytes);
        *v.status = ok;
        if (s.status_out) s.status_out[r] = ok;
        if (!ok && b.fail_count) add_u32(b.fail_count, 1);
    }
}

}  // namespace

hipError_t launch_gcm(int mode, hipStream_t stream, const GcmCtx* ctx, const RecBatch& b, const Sched& s, RecAcc*,
                      bool, const LaunchEvents&)
{
    if (b.single || mode < 0 || mode > 2) return hipErrorInvalidValue;  // the host runtime launches layers only
    auto bb = std::make_shared<RecBatch>(b);
    auto ss = std::make_shared<Sched>(s);
    S(stream)->push([mode, ctx, bb, ss] { layer_kernel(mode, ctx, *bb, *ss); });
    return hipSuccess;
}

hipError_t launch_release(hipStream_t stream, const GcmCtx* ctx, const RecBatch& b, uint32_t nrec, uint64_t bytes,
                          bool, const uint32_t* gate, uint32_t, const LaunchEvents&)
{
    S(stream)->push([ctx, b, nrec, bytes, gate] {
        if (gated(gate)) return;
        uint8_t key[16];
        key_of(ctx, key);
        for (uint32_t r = 0; r < nrec; ++r) {
            const View v = view(b, r);
            if (v.skip) continue;
            if (*v.status == 1u && !v.bad) ctr(key, v.iv12, v.src, bytes, v.dst);
            else memset(v.dst, 0, bytes);
        }
    });
    return hipSuccess;
}

hipError_t launch_dequant_scatter(hipStream_t stream, const CodecBatch& b, const LaunchEvents&)
{
    S(stream)->push([b] {
        if (gated(b.gate)) return;
        for (uint32_t r = 0; r < b.nrec; ++r) {
            const int64_t sid = b.slots[r];
            if (sid < 0 || sid >= b.nslots) continue;
            const uint32_t kind = r < b.n_k ? 0u : 1u;
            si_or_codec_decode(b.staging + uint64_t(r) * b.staging_stride, b.heads, b.dim, b.bits, kind,
                               reinterpret_cast<uint16_t*>(b.cache[kind] + uint64_t(sid) * b.slot_bytes));
        }
    });
    return hipSuccess;
}

hipError_t launch_gather_quant(hipStream_t stream, const CodecBatch& b, const LaunchEvents&)
{
    S(stream)->push([b] {
        std::vector<uint16_t> zero(size_t(128) * b.heads * b.dim, 0);
        for (uint32_t r = 0; r < b.nrec; ++r) {
            const int64_t sid = b.slots[r];
            const uint32_t kind = r < b.n_k ? 0u : 1u;
            const uint16_t* blk = (sid < 0 || sid >= b.nslots)
                                      ? zero.data()
                                      : reinterpret_cast<const uint16_t*>(b.cache[kind] + uint64_t(sid) * b.slot_bytes);
            si_or_codec_encode(blk, b.heads, b.dim, b.bits, kind, b.layer, b.staging + uint64_t(r) * b.staging_stride);
        }
    });
    return hipSuccess;
}

uint8_t* noalloc_scratch(hipStream_t)
{
    static uint8_t* p = static_cast<uint8_t*>(calloc(1, SI_NOALLOC_SCRATCH_BYTES));
    return p;
}

hipError_t launch_noalloc_acquire(hipStream_t stream, uint32_t* ctrl, uint32_t* cell)
{
    S(stream)->push([ctrl, cell] {
        uint32_t tok;
        do {
            tok = __atomic_add_fetch(&ctrl[1], 1u, __ATOMIC_SEQ_CST);
        } while (tok == 0u || tok == SI_NOALLOC_TEST_TOKEN);
        uint32_t expected = 0;
        const bool won = __atomic_compare_exchange_n(&ctrl[0], &expected, tok, false, __ATOMIC_SEQ_CST,
                                                     __ATOMIC_SEQ_CST);
        __atomic_store_n(cell, won ? tok : 0u, __ATOMIC_SEQ_CST);
    });
    return hipSuccess;
}

hipError_t launch_noalloc_finish(hipStream_t stream, const NoallocFinish& f)
{
    S(stream)->push([f] {
        const uint32_t tok = __atomic_load_n(f.cell, __ATOMIC_SEQ_CST);
        if (tok) {
            uint32_t expected = tok;
            __atomic_compare_exchange_n(&f.ctrl[0], &expected, 0u, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
            return;
        }
        for (uint32_t r = 0; r < f.nrec; ++r) {
            *reinterpret_cast<uint32_t*>(f.wire + uint64_t(r) * f.wire_stride + f.status_off) = 0;
            if (f.status_out) f.status_out[r] = 0;
            const int64_t sid = f.slots[r];
            if (sid >= 0 && sid < f.nslots)
                memset(f.cache[r < f.n_k ? 0 : 1] + uint64_t(sid) * f.slot_bytes, 0, f.out_bytes);
        }
        if (f.fail_count) add_u32(f.fail_count, f.nrec);
    });
    return hipSuccess;
}

hipError_t launch_noalloc_test_hold(hipStream_t stream, uint32_t* ctrl, int hold)
{
    S(stream)->push([ctrl, hold] {
        uint32_t expected = hold ? 0u : SI_NOALLOC_TEST_TOKEN;
        __atomic_compare_exchange_n(&ctrl[0], &expected, hold ? SI_NOALLOC_TEST_TOKEN : 0u, false, __ATOMIC_SEQ_CST,
                                    __ATOMIC_SEQ_CST);
    });
    return hipSuccess;
}

// Not launched by the host runtime: the kernel-level mirrors and the session
// agreement are exercised on the GPU only.
hipError_t launch_ctr(hipStream_t, const GcmCtx*, const uint8_t*, uint8_t*, uint64_t, const uint32_t*)
{
    return hipErrorInvalidValue;
}
hipError_t launch_auth_gate(hipStream_t, uint8_t*, const uint32_t*, uint64_t) { return hipErrorInvalidValue; }
hipError_t launch_ghash(hipStream_t, const GcmCtx*, const GhashJob&) { return hipErrorInvalidValue; }
hipError_t launch_agree(hipStream_t, const uint8_t*, const uint8_t*, const AgreeSeed&, uint32_t*, uint32_t*, uint8_t*,
                        uint8_t*, uint8_t*, int32_t*)
{
    return hipErrorInvalidValue;
}
hipError_t launch_ctx_build(hipStream_t, const uint8_t*, const uint32_t*, GcmCtx*, uint32_t)
{
    return hipErrorInvalidValue;
}
hipError_t launch_zero_bytes(hipStream_t, uint8_t*, uint32_t) { return hipErrorInvalidValue; }
hipError_t launch_x25519_test(hipStream_t, const uint8_t*, const uint8_t*, uint8_t*) { return hipErrorInvalidValue; }
hipError_t launch_blake2b_test(hipStream_t, const uint8_t*, uint32_t, const uint8_t*, uint64_t, uint8_t*, uint32_t)
{
    return hipErrorInvalidValue;
}

}  // namespace si

// Takes the reload log of one layer out of the log (layer numbers come back
// in later rounds): rows of (kind, block id, ticket); returns the count (at
// most cap rows written).
extern "C" size_t hostsim_reload_log(uint32_t layer, uint64_t* out, size_t cap)
{
    std::lock_guard<std::mutex> g(si::g_log_m);
    size_t n = 0;
    auto keep = si::g_log.begin();
    for (auto it = si::g_log.begin(); it != si::g_log.end(); ++it) {
        const auto e = *it;
        if (e[0] != layer) {
            *keep++ = e;
            continue;
        }
        if (n < cap) {
            out[3 * n] = e[1];
            out[3 * n + 1] = e[2];
            out[3 * n + 2] = e[3];
        }
        ++n;
    }
    si::g_log.erase(keep, si::g_log.end());
    return n;
}
