// Host side of the authenticated transfer path on MI355X.
//
//  * A worker pool runs OpenSSL AES-128-GCM (EVP, one context per thread) --
//    the reference's host crypto (inline_h2d_encrypt_commit,
//    secure_infer.cpp:6486-6550; d2h_host_decrypt_one, :2470-2547).  Idle
//    workers poll for work for SECURE_INFER_POOL_SPIN_US (default 200) before
//    they park.
//  * H2D: secure_infer_h2d_swap seals host KV blocks into wire records in a
//    pinned ring slot of the caller's stream, copies the slot to the device
//    on that ring's copy stream and makes the caller's stream wait for the
//    copy before the fused verify + decrypt (+ dequant) + paged-scatter
//    kernel.  The caller returns as soon as the work is queued, so the copy
//    of layer l+1 overlaps the kernel of layer l.  Inside a layer group the
//    swaps' records accumulate in one ring slot and go out as one copy
//    sequence and one launch at the group's end (K swaps before V swaps of
//    one stream), as the reference batches a group's swaps
//    (secure_infer.cpp:5862-5904): each cross-stream wait and launch costs
//    the host about 10 us in the HIP runtime.  Rings, their copy streams and
//    their locks are per (device, caller stream), like the reference's
//    per-stream pipelines (:5389-5399).
//  * Observation and strict retry: inside a layer group the kernel also
//    stores every record's status into mapped pinned host memory, read once
//    an event after the kernel has completed (observe_recovery_authentication,
//    secure_infer.cpp:5316-5387);
//    secure_infer_recovery_wait_layer_authentication re-seals a record that
//    failed once from the trusted host copy under a fresh ticket and
//    returns -1 only when that second attempt fails too (:7303-7333).
//  * D2H: the reference's batch / group API with the same names and
//    thread-local contexts (secure_infer.cpp:2707-2970).  A batch's swaps of
//    one stream and layer accumulate into one launch (gather + quantise +
//    seal on the caller's stream, records copied to pinned memory on a D2H
//    stream); a per-device watcher thread hands each launch to the worker
//    pool once its copy is done, which authenticates and decrypts each
//    record into its host destination (a record that fails is zeroed).
//    Launches in flight are bounded; batch_end waits for the verification.
//  * Ahead-of-demand sealing (the reference's CPU ciphertext prefetch,
//    secure_infer.cpp:3264-3710): secure_infer_h2d_prefetch seals a swap's
//    records on the worker pool before the swap is issued, under tickets
//    reserved then; the matching secure_infer_h2d_swap only copies them.
//  * An optional per-launch ledger (SECURE_INFER_H2D_PROFILE=<csv path>) of
//    host seal time, H2D copy time and kernel time, like the reference's
//    per-copy profile rows (secure_infer.cpp:1826-1951, 6085-6137).
//  * Every block id is range-checked on the host before any work: a swap
//    with a host block or device slot outside its pool is refused (-1).
#include "si_host.h"

#include <openssl/evp.h>
#include <sched.h>

#include <algorithm>
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
#include <unordered_map>
#include <vector>

namespace {

void put_be64(uint8_t* p, uint64_t v)
{
    for (int i = 0; i < 8; ++i) p[i] = uint8_t(v >> (56 - 8 * i));
}

// ---------------------------------------------------------------- worker pool

class Pool {
public:
    static Pool& get()
    {
        static Pool* p = new Pool();  // never destroyed: workers may be parked at exit
        return *p;
    }

    void submit(std::function<void()> f)
    {
        {
            std::lock_guard<std::mutex> g(m_);
            q_.push_back(std::move(f));
            queued_.fetch_add(1, std::memory_order_release);
        }
        cv_.notify_one();
    }

    // Queues every task under one lock with one wake-up.
    void submit_all(std::vector<std::function<void()>>& fs)
    {
        if (fs.empty()) return;
        {
            std::lock_guard<std::mutex> g(m_);
            for (auto& f : fs) q_.push_back(std::move(f));
            queued_.fetch_add(fs.size(), std::memory_order_release);
        }
        fs.clear();
        cv_.notify_all();
    }

    // f(i) for every i in [0, n), on the pool and the calling thread.
    void parallel_for(size_t n, const std::function<void(size_t)>& f)
    {
        if (n == 0) return;
        struct Shared {
            std::atomic<size_t> next{0}, done{0};
            std::mutex m;
            std::condition_variable cv;
        };
        auto sh = std::make_shared<Shared>();
        const std::function<void(size_t)>* fp = &f;
        auto body = [sh, n, fp]() {
            for (size_t i; (i = sh->next.fetch_add(1)) < n;) {
                (*fp)(i);
                if (sh->done.fetch_add(1) + 1 == n) {
                    std::lock_guard<std::mutex> g(sh->m);
                    sh->cv.notify_all();
                }
            }
        };
        // One lock and one wake-up for all helpers: a futex wake per helper
        // costs the caller more than a 41-KB record's seal.
        const size_t helpers = std::min(threads_.size(), n - 1);
        if (helpers) {
            {
                std::lock_guard<std::mutex> g(m_);
                for (size_t h = 0; h < helpers; ++h) q_.push_back(body);
                queued_.fetch_add(helpers, std::memory_order_release);
            }
            if (helpers == 1)
                cv_.notify_one();
            else
                cv_.notify_all();
        }
        body();
        spin_until([&] { return sh->done.load(std::memory_order_acquire) == n; });
        std::unique_lock<std::mutex> g(sh->m);
        sh->cv.wait(g, [&] { return sh->done.load() == n; });
    }

    size_t threads() const { return threads_.size() + 1; }

private:
    Pool()
    {
        // CPUs this process may run on (the affinity mask, not the machine),
        // less one that stays free for the HIP runtime's own threads (they
        // submit the ring's copies while the pool seals the next swap).
        unsigned n = std::thread::hardware_concurrency();
        cpu_set_t set;
        CPU_ZERO(&set);
        if (sched_getaffinity(0, sizeof(set), &set) == 0) n = unsigned(CPU_COUNT(&set));
        if (n > 2) n -= 1;
        if (const char* e = std::getenv("SECURE_INFER_HOST_THREADS")) n = unsigned(std::atoi(e));
        if (n == 0) n = 1;
        if (n > 256) n = 256;
        if (const char* e = std::getenv("SECURE_INFER_POOL_SPIN_US")) spin_us_ = std::max(0, std::atoi(e));
        for (unsigned i = 0; i + 1 < n; ++i) threads_.emplace_back([this] { run(); });
    }

    // Polls `ready` for up to spin_us_ before the caller blocks: a transfer's
    // swaps arrive tens of microseconds apart, about what waking a thread
    // parked on a futex costs, so idle workers (and a caller waiting for its
    // helpers) poll for a while first.
    template <class F>
    void spin_until(F ready) const
    {
        if (spin_us_ <= 0 || ready()) return;
        const auto until = std::chrono::steady_clock::now() + std::chrono::microseconds(spin_us_);
        for (unsigned i = 1; !ready(); ++i) {
#if defined(__x86_64__)
            __builtin_ia32_pause();
#endif
            if ((i & 63) == 0 && std::chrono::steady_clock::now() >= until) return;
        }
    }

    void run()
    {
        for (;;) {
            spin_until([&] { return queued_.load(std::memory_order_acquire) != 0; });
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> g(m_);
                cv_.wait(g, [&] { return !q_.empty(); });
                f = std::move(q_.front());
                q_.pop_front();
                queued_.fetch_sub(1, std::memory_order_relaxed);
            }
            f();
        }
    }

    std::vector<std::thread> threads_;
    std::deque<std::function<void()>> q_;
    std::atomic<size_t> queued_{0};
    int spin_us_ = 200;
    std::mutex m_;
    std::condition_variable cv_;
};

// ---------------------------------------------------------------- OpenSSL GCM

EVP_CIPHER_CTX* thread_ctx()
{
    thread_local std::unique_ptr<EVP_CIPHER_CTX, void (*)(EVP_CIPHER_CTX*)> c(EVP_CIPHER_CTX_new(),
                                                                              EVP_CIPHER_CTX_free);
    return c.get();
}

const size_t kChunk = size_t(1) << 30;  // EVP lengths are int

bool gcm_seal(const uint8_t key[16], const uint8_t iv[12], const uint8_t* aad, size_t aad_len,
              const uint8_t* in, size_t n, uint8_t* out, uint8_t tag[16])
{
    EVP_CIPHER_CTX* c = thread_ctx();
    int len = 0;
    if (!c || EVP_EncryptInit_ex(c, EVP_aes_128_gcm(), nullptr, nullptr, nullptr) != 1 ||
        EVP_CIPHER_CTX_ctrl(c, EVP_CTRL_GCM_SET_IVLEN, 12, nullptr) != 1 ||
        EVP_EncryptInit_ex(c, nullptr, nullptr, key, iv) != 1)
        return false;
    if (aad_len && EVP_EncryptUpdate(c, nullptr, &len, aad, int(aad_len)) != 1) return false;
    for (size_t o = 0; o < n; o += kChunk) {
        const int k = int(std::min(kChunk, n - o));
        if (EVP_EncryptUpdate(c, out + o, &len, in + o, k) != 1) return false;
    }
    if (EVP_EncryptFinal_ex(c, out + n, &len) != 1) return false;
    return EVP_CIPHER_CTX_ctrl(c, EVP_CTRL_GCM_GET_TAG, 16, tag) == 1;
}

// Authenticated decryption; false on a tag mismatch (out then holds garbage).
bool gcm_open(const uint8_t key[16], const uint8_t iv[12], const uint8_t* aad, size_t aad_len,
              const uint8_t* in, size_t n, const uint8_t tag[16], uint8_t* out)
{
    EVP_CIPHER_CTX* c = thread_ctx();
    int len = 0;
    if (!c || EVP_DecryptInit_ex(c, EVP_aes_128_gcm(), nullptr, nullptr, nullptr) != 1 ||
        EVP_CIPHER_CTX_ctrl(c, EVP_CTRL_GCM_SET_IVLEN, 12, nullptr) != 1 ||
        EVP_DecryptInit_ex(c, nullptr, nullptr, key, iv) != 1)
        return false;
    if (aad_len && EVP_DecryptUpdate(c, nullptr, &len, aad, int(aad_len)) != 1) return false;
    for (size_t o = 0; o < n; o += kChunk) {
        const int k = int(std::min(kChunk, n - o));
        if (EVP_DecryptUpdate(c, out + o, &len, in + o, k) != 1) return false;
    }
    if (EVP_CIPHER_CTX_ctrl(c, EVP_CTRL_GCM_SET_TAG, 16, const_cast<uint8_t*>(tag)) != 1) return false;
    return EVP_DecryptFinal_ex(c, out + n, &len) > 0;
}

void record_iv(const si_internal::SessionKeys& k, uint64_t ticket, uint8_t iv[12])
{
    memcpy(iv, k.salt, 4);
    put_be64(iv + 4, k.nonce + ticket);
}

uint64_t tag_offset(uint64_t bytes) { return (bytes + 31) & ~uint64_t(31); }

// ---------------------------------------------------------------- test fault injection
//
// The reference's opt-in, test-only bit flips at the two trust boundaries:
// after the host sealed an H2D record and before its DMA
// (PIPE_GCM_TAMPER_H2D*, secure_infer.cpp:6139-6250), and after a D2H record
// reached host memory and before host authentication (PIPE_GCM_TAMPER_D2H,
// :2451-2467).  Disarmed unless a test arms them.

struct H2DTamper {
    std::atomic<int64_t> layer{-1}, kind{-1}, block{-1};
    std::atomic<int64_t> shots{0};
};
H2DTamper g_tamper_h2d;
std::atomic<int64_t> g_tamper_d2h{0};

bool take_shot(std::atomic<int64_t>& shots)
{
    int64_t s = shots.load();
    while (s > 0)
        if (shots.compare_exchange_weak(s, s - 1)) return true;
    return false;
}

bool tamper_h2d(uint32_t layer, uint32_t kind, int64_t host_block)
{
    if (g_tamper_h2d.shots.load() <= 0) return false;
    const int64_t l = g_tamper_h2d.layer.load(), k = g_tamper_h2d.kind.load(), b = g_tamper_h2d.block.load();
    if ((l >= 0 && l != int64_t(layer)) || (k >= 0 && k != int64_t(kind)) || (b >= 0 && b != host_block))
        return false;
    return take_shot(g_tamper_h2d.shots);
}

// ---------------------------------------------------------------- device buffers

struct Prefetch;

// One ledger row of an H2D launch (or, in records mode, one row per record),
// written once its slot's work is complete.
struct ProfileRow {
    bool pending = false;
    uint32_t layer = 0, kind = 0, n = 0, source = 0;  // source: 0 sealed on demand, 1 prefetched, 2 waited
    uint64_t bytes = 0, stride = 0;
    double seal_us = 0;
    double copy_enqueue_us = 0, kernel_enqueue_us = 0;  // host time issuing the launch's copies / kernels
    std::vector<float> rec_seal_us;       // records mode: each record's own seal, device order
    std::vector<uint8_t> rec_prefetched;  // ... and whether it was sealed ahead of demand
};

// A pinned host buffer mirrored by a device buffer of the same size, plus
// device scratch for codec packets, reused across calls.
struct Mirror {
    uint8_t* host = nullptr;
    uint8_t* dev = nullptr;
    size_t cap = 0;
    uint8_t* stage = nullptr;
    size_t stage_cap = 0;
    hipEvent_t ev_a = nullptr;  // H2D: wire records landed; D2H: records sealed
    hipEvent_t ev_b = nullptr;  // H2D: slot free again; D2H: records in host memory
    // ledger (timing events, created when the ledger is on)
    hipEvent_t p_c0 = nullptr, p_c1 = nullptr, p_k0 = nullptr, p_k1 = nullptr;
    ProfileRow row;
    std::vector<std::shared_ptr<Prefetch>> held;  // prefetched records being copied from

    Mirror() = default;
    Mirror(const Mirror&) = delete;
    Mirror& operator=(const Mirror&) = delete;
    // Only reached for buffers no queued work refers to (failed set-up).
    ~Mirror()
    {
        if (host) (void)hipHostFree(host);
        if (dev) (void)hipFree(dev);
        if (stage) (void)hipFree(stage);
        if (ev_a) (void)hipEventDestroy(ev_a);
        if (ev_b) (void)hipEventDestroy(ev_b);
        for (hipEvent_t e : {p_c0, p_c1, p_k0, p_k1})
            if (e) (void)hipEventDestroy(e);
    }

    bool init_profile()
    {
        if (p_c0) return true;
        return hipEventCreate(&p_c0) == hipSuccess && hipEventCreate(&p_c1) == hipSuccess &&
               hipEventCreate(&p_k0) == hipSuccess && hipEventCreate(&p_k1) == hipSuccess;
    }

    bool init()
    {
        return hipEventCreateWithFlags(&ev_a, hipEventDisableTiming) == hipSuccess &&
               hipEventCreateWithFlags(&ev_b, hipEventDisableTiming) == hipSuccess;
    }
    // Callers guarantee no queued work still uses the buffers.
    bool reserve(size_t need, size_t stage_need)
    {
        if (need > cap) {
            if (host) (void)hipHostFree(host);
            if (dev) (void)hipFree(dev);
            host = nullptr;
            dev = nullptr;
            cap = 0;
            if (hipHostMalloc(reinterpret_cast<void**>(&host), need, hipHostMallocDefault) != hipSuccess ||
                hipMalloc(reinterpret_cast<void**>(&dev), need) != hipSuccess)
                return false;
            cap = need;
        }
        if (stage_need > stage_cap) {
            if (stage) (void)hipFree(stage);
            stage = nullptr;
            stage_cap = 0;
            if (hipMalloc(reinterpret_cast<void**>(&stage), stage_need) != hipSuccess) return false;
            stage_cap = stage_need;
        }
        return true;
    }
};

// Pinned status words of one observed swap and the event after their copy.
// Per-record statuses of one observed swap: pinned, coherent host memory the
// reload kernel's finalisers store into directly (`dev` is its device-side
// address), readable on the host once `ready` (recorded after the kernel)
// has completed.
struct StatusBuf {
    uint32_t* host = nullptr;
    uint32_t* dev = nullptr;
    size_t cap = 0;  // words
    hipEvent_t ready = nullptr;
    bool orphaned = false;  // a failed launch may still store into it: never reused
    ~StatusBuf()
    {
        if (host) (void)hipHostFree(host);
        if (ready) (void)hipEventDestroy(ready);
    }
};

// The reload ring of one caller stream: slots, their cursor and lock, and
// the copy stream of its H2D records.
struct StreamRing {
    std::mutex lock;
    hipStream_t copy = nullptr;
    std::vector<std::unique_ptr<Mirror>> slots;
    std::vector<bool> used;  // a launch was issued from the slot (wait for its ev_b)
    std::vector<bool> busy;  // a pending launch is filling the slot
    size_t next = 0;
};

struct DeviceState {
    int device = 0;
    hipStream_t d2h = nullptr;  // D2H copies of sealed records
    std::mutex rings_lock;
    std::unordered_map<hipStream_t, std::unique_ptr<StreamRing>> rings;
    std::mutex pool_lock;
    std::vector<std::unique_ptr<Mirror>> free_bufs;  // D2H buffers not in flight
    std::condition_variable d2h_cv;                  // d2h_inflight went down (pool_lock)
    size_t d2h_inflight = 0;                         // bytes of D2H buffers in flight (pool_lock)
    size_t d2h_jobs = 0;                             // D2H launches in flight (pool_lock)
    struct D2HWatcher* watcher = nullptr;            // started by the first D2H launch
    std::mutex status_lock;
    std::vector<std::unique_ptr<StatusBuf>> free_status;
};

// The host runtime's registries are created once and never destroyed: the
// worker pool's threads, ring slots holding pinned and device buffers and
// pending prefetches may still refer to them while the process exits, after
// the HIP runtime has begun to tear down.
std::mutex g_states_lock;
std::map<int, std::unique_ptr<DeviceState>>& g_states = *new std::map<int, std::unique_ptr<DeviceState>>();

DeviceState* device_state()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> g(g_states_lock);
    auto& st = g_states[dev];
    if (!st) {
        auto s = std::make_unique<DeviceState>();
        s->device = dev;
        // default priority on purpose: every stream of the library shares it
        if (hipStreamCreateWithFlags(&s->d2h, hipStreamNonBlocking) != hipSuccess) return nullptr;
        st = std::move(s);
    }
    return st.get();
}

StreamRing* ring_of(DeviceState* ds, hipStream_t stream)
{
    std::lock_guard<std::mutex> g(ds->rings_lock);
    auto& r = ds->rings[stream];
    if (!r) {
        auto nr = std::make_unique<StreamRing>();
        if (hipStreamCreateWithFlags(&nr->copy, hipStreamNonBlocking) != hipSuccess) return nullptr;
        // Slots per stream: a layer of 16-block causal groups is 6 swaps, and
        // a slot is reused only after its kernel is done
        // (the reference's default budget is 32 single-record slots,
        // secure_infer.cpp:5608-5647).
        size_t slots = 16;
        if (const char* e = std::getenv("SECURE_INFER_H2D_SLOTS")) slots = size_t(std::max(2, std::atoi(e)));
        for (size_t i = 0; i < slots; ++i) {
            auto mbuf = std::make_unique<Mirror>();
            if (!mbuf->init()) return nullptr;
            nr->slots.push_back(std::move(mbuf));
            nr->used.push_back(false);
            nr->busy.push_back(false);
        }
        r = std::move(nr);
    }
    return r.get();
}

// A status buffer of at least `words` entries, all 0 (failed) until the
// kernel stores each record's result.  Buffers come back to the free list
// only after their `ready` event has completed, so no kernel still writes them.
std::unique_ptr<StatusBuf> take_status(DeviceState* ds, size_t words)
{
    {
        std::lock_guard<std::mutex> g(ds->status_lock);
        for (size_t i = 0; i < ds->free_status.size(); ++i)
            if (ds->free_status[i]->cap >= words) {
                auto b = std::move(ds->free_status[i]);
                ds->free_status.erase(ds->free_status.begin() + long(i));
                memset(b->host, 0, words * 4);
                return b;
            }
    }
    auto b = std::make_unique<StatusBuf>();
    const size_t cap = std::max<size_t>(1024, (words + 1023) / 1024 * 1024);
    if (hipHostMalloc(reinterpret_cast<void**>(&b->host), cap * 4, hipHostMallocDefault) != hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void**>(&b->dev), b->host, 0) != hipSuccess ||
        hipEventCreateWithFlags(&b->ready, hipEventDisableTiming) != hipSuccess)
        return nullptr;
    memset(b->host, 0, cap * 4);
    b->cap = cap;
    return b;
}

void give_status(DeviceState* ds, std::unique_ptr<StatusBuf> b)
{
    if (!b) return;
    std::lock_guard<std::mutex> g(ds->status_lock);
    ds->free_status.push_back(std::move(b));
}

bool valid_geometry(uint32_t codec, uint32_t heads, uint32_t dim, uint64_t host_block_bytes,
                    uint64_t& bytes)
{
    if (codec == SI_CODEC_NONE) {
        bytes = host_block_bytes;
        return bytes > 0;
    }
    if (codec != SI_CODEC_INT8 && codec != SI_CODEC_INT4) return false;
    if (heads == 0 || dim == 0 || dim % 64) return false;
    bytes = secure_infer_codec_width(codec, heads, dim);
    return host_block_bytes >= bytes;
}

// Every (host block, device slot) of a swap inside its pool.
bool valid_mapping(const int64_t* mapping, uint32_t n, bool host_first, uint64_t host_nblocks,
                   uint64_t nslots)
{
    for (uint32_t r = 0; r < n; ++r) {
        const int64_t hb = mapping[2 * r + (host_first ? 0 : 1)];
        const int64_t ds = mapping[2 * r + (host_first ? 1 : 0)];
        if (hb < 0 || uint64_t(hb) >= host_nblocks || ds < 0 || uint64_t(ds) >= nslots) return false;
    }
    return true;
}

// ---------------------------------------------------------------- H2D ledger

std::mutex g_profile_lock;
FILE* g_profile = nullptr;
bool g_profile_checked = false;

std::atomic<bool> g_profile_paused{false};

// SECURE_INFER_H2D_PROFILE_RECORDS=1: one row per record in the reference's
// per-copy column set (secure_infer.cpp:1846-1847, 5649-5690) instead of one
// row per launch.
bool profile_records()
{
    static const bool on = [] {
        const char* e = std::getenv("SECURE_INFER_H2D_PROFILE_RECORDS");
        return e && std::atoi(e) != 0;
    }();
    return on;
}

bool profile_on()
{
    if (g_profile_paused.load(std::memory_order_relaxed)) return false;
    std::lock_guard<std::mutex> g(g_profile_lock);
    if (!g_profile_checked) {
        g_profile_checked = true;
        const char* path = std::getenv("SECURE_INFER_H2D_PROFILE");
        if (path && *path) {
            g_profile = std::fopen(path, "a");
            if (g_profile && profile_records())
                std::fprintf(g_profile,
                             "direction,bytes,aligned_bytes,total_us,cpu_crypto_us,device_pipeline_us,host_wait_us,"
                             "copy_enqueue_us,kernel_enqueue_us,h2d_device_us,kernel_execute_us,d2d_device_us,"
                             "device_total_us,device_timing_valid,crypto_mode,cpu_prediction_hit\n");
            else if (g_profile)
                std::fprintf(g_profile, "layer,kind,records,record_bytes,source,seal_us,h2d_copy_us,kernel_us\n");
        }
    }
    return g_profile != nullptr;
}

// Writes the slot's pending row; its events must be complete.
void profile_retire(Mirror& sl)
{
    if (!sl.row.pending) return;
    sl.row.pending = false;
    float copy_ms = -1.0f, kernel_ms = -1.0f, total_ms = -1.0f;
    const bool valid = hipEventElapsedTime(&copy_ms, sl.p_c0, sl.p_c1) == hipSuccess &&
                       hipEventElapsedTime(&kernel_ms, sl.p_k0, sl.p_k1) == hipSuccess &&
                       hipEventElapsedTime(&total_ms, sl.p_c0, sl.p_k1) == hipSuccess;
    static const char* kSource[] = {"sealed", "prefetched", "prefetch_waited"};
    std::lock_guard<std::mutex> g(g_profile_lock);
    if (g_profile && profile_records()) {
        // Per record: its own seal on the host; the launch that carried it
        // (every record of it alike) for the enqueue times and the device
        // phases (copy start to copy end, kernel, copy start to kernel end).
        // No device-to-device stage follows the kernel, and a swap that
        // finds its records sealed ahead waits on nothing else.
        auto us = [](double x) { return static_cast<unsigned long long>(x < 0 ? 0 : x + 0.5); };
        const double dev = valid ? double(total_ms) * 1e3 : 0.0;
        for (size_t r = 0; r < sl.row.rec_seal_us.size(); ++r) {
            const double seal = sl.row.rec_seal_us[r];
            std::fprintf(g_profile, "H2D,%llu,%llu,%llu,%llu,%llu,0,%llu,%llu,%llu,%llu,0,%llu,%d,0,%d\n",
                         static_cast<unsigned long long>(sl.row.bytes), static_cast<unsigned long long>(sl.row.stride),
                         us(seal + sl.row.copy_enqueue_us + sl.row.kernel_enqueue_us + dev), us(seal), us(dev),
                         us(sl.row.copy_enqueue_us), us(sl.row.kernel_enqueue_us),
                         us(valid ? double(copy_ms) * 1e3 : 0.0), us(valid ? double(kernel_ms) * 1e3 : 0.0), us(dev),
                         valid ? 1 : 0, int(sl.row.rec_prefetched[r]));
        }
    } else if (g_profile)
        std::fprintf(g_profile, "%u,%u,%u,%llu,%s,%.1f,%.1f,%.1f\n", sl.row.layer, sl.row.kind, sl.row.n,
                     static_cast<unsigned long long>(sl.row.bytes), kSource[sl.row.source % 3], sl.row.seal_us,
                     double(copy_ms) * 1e3, double(kernel_ms) * 1e3);
}

// Retires the ledger rows of every ring slot whose work is done (wait:
// synchronise with the pending ones first), then flushes the file.
void profile_sweep(bool wait)
{
    std::vector<DeviceState*> states;
    {
        std::lock_guard<std::mutex> g(g_states_lock);
        for (auto& kv : g_states) states.push_back(kv.second.get());
    }
    for (DeviceState* ds : states) {
        std::vector<StreamRing*> rings;
        {
            std::lock_guard<std::mutex> g(ds->rings_lock);
            for (auto& kv : ds->rings) rings.push_back(kv.second.get());
        }
        for (StreamRing* ring : rings) {
            std::lock_guard<std::mutex> g(ring->lock);
            for (auto& sl : ring->slots) {
                if (!sl->row.pending) continue;
                const hipError_t st = wait ? hipEventSynchronize(sl->ev_b) : hipEventQuery(sl->ev_b);
                if (st == hipSuccess) profile_retire(*sl);
            }
        }
    }
    std::lock_guard<std::mutex> g(g_profile_lock);
    if (g_profile) std::fflush(g_profile);
}

// ---------------------------------------------------------------- ahead-of-demand sealing

// A swap's records sealed before the swap is issued: n wire records laid out
// as in a ring slot, in pinned memory, copied from there by the swap.  It
// serves the secure_infer_h2d_swap with the same session, host pool, kind,
// layer, codec and host-block column of the mapping.
struct Prefetch {
    si_session* session = nullptr;
    si_internal::SessionKeys keys{};
    const uint8_t* host_base = nullptr;
    uint64_t host_block_bytes = 0;
    uint32_t kind = 0, layer = 0, codec = 0, heads = 0, dim = 0, n = 0;
    std::vector<int64_t> host_blocks;
    uint64_t bytes = 0, stride = 0, tag_off = 0, t0 = 0;
    uint8_t* host = nullptr;
    size_t cap = 0;  // bytes of `host` this prefetch owns (0: a part of `owner`'s buffer)
    std::shared_ptr<Prefetch> owner;  // the K half of a group prefetch, whose buffer this shares
    // A group prefetch (K half): its buffer is [K records][V records][slot ids of
    // both halves], so one DMA can carry the group's launch.
    const uint8_t* group_ids = nullptr;
    uint32_t group_records = 0;
    // A layer prefetch (its first K part owns the buffer): [every group's K
    // records][every group's V records][IV words][slot ids], the device
    // layout of a launch of exactly the layer's swaps, so one DMA carries it.
    const uint8_t* layer_tail = nullptr;
    uint32_t layer_records = 0;
    std::mutex m;
    std::condition_variable cv;
    uint32_t tasks = 0, done = 0;
    bool failed = false;
    bool started = false;
    std::chrono::steady_clock::time_point first_start{};
    double seal_us = 0;  // first sealing task's start to the last one's end
    std::vector<float> rec_us;  // each record's seal (its own task)
    ~Prefetch();
};

std::mutex g_pf_lock;
std::vector<std::shared_ptr<Prefetch>>& g_prefetch = *new std::vector<std::shared_ptr<Prefetch>>();  // not consumed
std::vector<std::pair<uint8_t*, size_t>>& g_pf_free = *new std::vector<std::pair<uint8_t*, size_t>>();  // to reuse
size_t g_pf_bytes = 0;                                        // pinned bytes held by prefetches
std::atomic<uint64_t> g_pf_ready{0}, g_pf_waited{0}, g_pf_missing{0};

size_t prefetch_budget()
{
    static const size_t b = [] {
        size_t mb = 2048;
        if (const char* e = std::getenv("SECURE_INFER_PREFETCH_MB")) mb = size_t(std::max(0, std::atoi(e)));
        return mb << 20;
    }();
    return b;
}

Prefetch::~Prefetch()
{
    if (!host || !cap) return;
    std::lock_guard<std::mutex> g(g_pf_lock);
    g_pf_free.emplace_back(host, cap);
}

// A pinned buffer of at least `need` bytes: the smallest free one that fits,
// else a new one within the budget, after freeing free buffers too small to
// serve (none of them is read by a queued copy any more).
uint8_t* take_pf_buffer(size_t need, size_t& cap)
{
    std::vector<uint8_t*> drop;
    bool fits = true;
    {
        std::lock_guard<std::mutex> g(g_pf_lock);
        size_t best = g_pf_free.size();
        for (size_t i = 0; i < g_pf_free.size(); ++i)
            if (g_pf_free[i].second >= need && (best == g_pf_free.size() || g_pf_free[i].second < g_pf_free[best].second))
                best = i;
        if (best < g_pf_free.size()) {
            uint8_t* p = g_pf_free[best].first;
            cap = g_pf_free[best].second;
            g_pf_free.erase(g_pf_free.begin() + long(best));
            return p;
        }
        while (g_pf_bytes + need > prefetch_budget() && !g_pf_free.empty()) {
            drop.push_back(g_pf_free.back().first);
            g_pf_bytes -= g_pf_free.back().second;
            g_pf_free.pop_back();
        }
        fits = g_pf_bytes + need <= prefetch_budget();
        if (fits) g_pf_bytes += need;
    }
    for (uint8_t* p : drop) (void)hipHostFree(p);
    if (!fits) return nullptr;
    uint8_t* p = nullptr;
    if (hipHostMalloc(reinterpret_cast<void**>(&p), need, hipHostMallocDefault) != hipSuccess) {
        std::lock_guard<std::mutex> g(g_pf_lock);
        g_pf_bytes -= need;
        return nullptr;
    }
    cap = need;
    return p;
}

double us_since(std::chrono::steady_clock::time_point t0)
{
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
}

void seal_record(const si_internal::SessionKeys& keys, const uint8_t* src, uint64_t bytes, uint64_t tag_off,
                 uint64_t ticket, uint8_t* rec, uint32_t layer, uint32_t kind, int64_t hb, bool& ok);

// A prefetch of n records of one kind sealed into `host` (tickets set by the
// caller), not yet registered.
std::shared_ptr<Prefetch> new_prefetch(si_session* s, const si_internal::SessionKeys& keys, const void* host_base,
                                       uint64_t host_block_bytes, const int64_t* mapping, uint32_t n, uint32_t kind,
                                       uint32_t layer, uint32_t codec, uint32_t heads, uint32_t dim, uint64_t bytes,
                                       uint8_t* host)
{
    auto pf = std::make_shared<Prefetch>();
    pf->session = s;
    pf->keys = keys;
    pf->host_base = static_cast<const uint8_t*>(host_base);
    pf->host_block_bytes = host_block_bytes;
    pf->kind = kind;
    pf->layer = layer;
    pf->codec = codec;
    pf->heads = heads;
    pf->dim = dim;
    pf->n = n;
    pf->bytes = bytes;
    pf->stride = secure_infer_wire_stride(bytes);
    pf->tag_off = tag_offset(bytes);
    pf->host_blocks.resize(n);
    for (uint32_t r = 0; r < n; ++r) pf->host_blocks[r] = mapping[2 * r];
    pf->rec_us.assign(n, 0.0f);
    pf->host = host;
    return pf;
}

// Registers the prefetch for its swap and appends its sealing tasks, one
// record per task (the pool balances records, not swaps).
void queue_seals(const std::shared_ptr<Prefetch>& pf, std::vector<std::function<void()>>& tasks)
{
    pf->tasks = pf->n;
    {
        std::lock_guard<std::mutex> g(g_pf_lock);
        g_prefetch.push_back(pf);
    }
    for (uint32_t r = 0; r < pf->n; ++r) {
        tasks.emplace_back([pf, r] {
            {
                std::lock_guard<std::mutex> g(pf->m);
                if (!pf->started) {
                    pf->started = true;
                    pf->first_start = std::chrono::steady_clock::now();
                }
            }
            bool ok = true;
            const int64_t hb = pf->host_blocks[r];
            const auto ts = std::chrono::steady_clock::now();
            seal_record(pf->keys, pf->host_base + uint64_t(hb) * pf->host_block_bytes, pf->bytes, pf->tag_off,
                        pf->t0 + r, pf->host + uint64_t(r) * pf->stride, pf->layer, pf->kind, hb, ok);
            pf->rec_us[r] = float(us_since(ts));
            std::lock_guard<std::mutex> g(pf->m);
            if (!ok) pf->failed = true;
            if (++pf->done == pf->tasks) {
                pf->seal_us = us_since(pf->first_start);
                pf->cv.notify_all();
            }
        });
    }
}

void wait_sealed(Prefetch& pf)
{
    std::unique_lock<std::mutex> g(pf.m);
    pf.cv.wait(g, [&] { return pf.done == pf.tasks; });
}

// The unconsumed prefetch that serves this swap, removed from the registry.
std::shared_ptr<Prefetch> take_prefetch(si_session* s, const void* host_base, uint64_t host_block_bytes,
                                        const int64_t* mapping, uint32_t n, uint32_t kind, uint32_t layer,
                                        uint32_t codec)
{
    std::lock_guard<std::mutex> g(g_pf_lock);
    for (size_t i = 0; i < g_prefetch.size(); ++i) {
        Prefetch& pf = *g_prefetch[i];
        if (pf.session != s || pf.host_base != host_base || pf.host_block_bytes != host_block_bytes ||
            pf.n != n || pf.kind != kind || pf.layer != layer || pf.codec != codec)
            continue;
        bool same = true;
        for (uint32_t r = 0; r < n && same; ++r) same = pf.host_blocks[r] == mapping[2 * r];
        if (!same) continue;
        auto out = g_prefetch[i];
        g_prefetch.erase(g_prefetch.begin() + long(i));
        return out;
    }
    return nullptr;
}

// ---------------------------------------------------------------- observed reloads

// Statuses shared by the swaps of one launch.  The buffer returns to its
// device's free list when the last swap lets go of it -- after its `ready`
// event completed -- unless a launch failed part-way and a kernel may still
// store into it (then it is never reused).
using StatusRef = std::shared_ptr<StatusBuf>;

StatusRef share_status(DeviceState* ds, std::unique_ptr<StatusBuf> b)
{
    if (!b) return nullptr;
    return StatusRef(b.release(), [ds](StatusBuf* p) {
        if (p->orphaned) return;
        give_status(ds, std::unique_ptr<StatusBuf>(p));
    });
}

// One observed swap: where each record came from and went to (for a strict
// retry from the trusted host copy) and where its statuses are.
struct Observed {
    DeviceState* ds = nullptr;
    si_session* session = nullptr;
    const uint8_t* host_base = nullptr;
    uint64_t host_block_bytes = 0, host_nblocks = 0;
    void* dev_cache = nullptr;
    uint64_t slot_bytes = 0, nslots = 0;
    uint32_t kind = 0, layer = 0, codec = 0, heads = 0, dim = 0;
    hipStream_t stream = nullptr;
    uint64_t job_id = 0;
    std::vector<int64_t> mapping;  // n (host block, device slot) pairs
    StatusRef status;
    uint32_t status_off = 0;       // the swap's first record among the launch's statuses
    uint32_t status_of(uint32_t r) const { return status->host[status_off + r]; }
};

std::mutex g_obs_lock;
std::multimap<uint32_t, std::shared_ptr<Observed>>& g_observed = *new std::multimap<uint32_t, std::shared_ptr<Observed>>();

// Observed swaps that nobody waits for would hold their status buffers
// forever: past kObservedSweep entries, swaps whose kernel has completed and
// whose every record authenticated are dropped (a wait would find nothing to
// report for them); failed and unfinished ones stay until waited for.
constexpr size_t kObservedSweep = 4096;

void sweep_observed_locked()
{
    if (g_observed.size() < kObservedSweep) return;
    for (auto it = g_observed.begin(); it != g_observed.end();) {
        const Observed& ob = *it->second;
        bool drop = hipEventQuery(ob.status->ready) == hipSuccess;
        for (uint32_t r = 0, n = uint32_t(ob.mapping.size() / 2); drop && r < n; ++r)
            drop = ob.status_of(r) == 1u;
        it = drop ? g_observed.erase(it) : std::next(it);
    }
}

// ---------------------------------------------------------------- H2D

void seal_record(const si_internal::SessionKeys& keys, const uint8_t* src, uint64_t bytes, uint64_t tag_off,
                 uint64_t ticket, uint8_t* rec, uint32_t layer, uint32_t kind, int64_t hb, bool& ok)
{
    uint8_t* aad = rec + tag_off + 32;
    uint8_t iv[12];
    record_iv(keys, ticket, iv);
    if (secure_infer_build_gcm_aad(src, bytes, 1, ticket, 0, keys.nonce, aad) != 1 ||
        !gcm_seal(keys.key, iv, aad, 64, src, bytes, rec, rec + tag_off)) {
        ok = false;
        return;
    }
    memset(rec + bytes, 0, tag_off - bytes);
    memset(rec + tag_off + 16, 0, 16);  // status slot
    if (tamper_h2d(layer, kind, hb)) rec[0] ^= 0x01;
}

// One swap's records within a launch.
struct H2DPart {
    const uint8_t* src = nullptr;  // its sealed records: ring slot rows or a prefetch buffer
    uint32_t r0 = 0, n = 0;        // host rows [r0, r0 + n) of the slot (swap order)
    uint32_t kind = 0;
    uint32_t dev_r0 = 0;           // first record on the device (K parts, then V parts)
    size_t ids0 = 0;               // its slot ids in the launch's slot_ids (swap order)
    uint64_t t0 = 0;               // ticket of its first record
    uint32_t source = 0;           // 0 sealed on demand, 1 prefetched, 2 prefetch waited for
    double seal_us = 0;
    std::vector<float> rec_us;     // ledger records mode: each record's seal
    std::shared_ptr<Prefetch> pf;
    std::shared_ptr<Observed> ob;  // null when not observed
};

// The records of consecutive swaps that go to the device as one copy
// sequence and one reload launch: all of one stream, session, layer and
// geometry.  On the host a ring slot holds them in swap order; on the device
// the launch is laid out [cap wire records: K parts, then V parts, each in
// swap order][iv words, n x 16][slot ids, n x 8], so K and V swaps may come
// in any order (a layer group around several causal groups takes K1 V1 K2
// V2 ...).  Inside a layer group the swaps accumulate until the group ends
// (or the next swap does not fit), as the reference batches a group's swaps
// (enqueue_h2d_gcm_batch_task, flushed by secure_infer_h2d_layer_group_end,
// secure_infer.cpp:5862-5904); outside a group every swap is a launch of
// its own.
struct H2DLaunch {
    hipStream_t stream = nullptr;
    si_session* s = nullptr;
    si_internal::SessionHold hold;  // until the launch is issued or dropped
    si_internal::SessionKeys keys{};
    DeviceState* ds = nullptr;
    StreamRing* ring = nullptr;
    size_t slot = 0;
    uint32_t layer = 0, codec = 0, heads = 0, dim = 0;
    uint64_t bytes = 0, stride = 0, tag_off = 0, slot_bytes = 0, nslots = 0;
    void* cache[2] = {nullptr, nullptr};
    uint32_t* fail_count = nullptr;
    bool observe = false;
    uint32_t cap = 0, n = 0, n_k = 0;
    std::vector<int64_t> slot_ids;
    std::vector<H2DPart> parts;
    StatusRef status;
};

void release_slot(StreamRing* ring, size_t idx, bool launched);

// The calling thread's pending launch.  A thread that ends with one (a layer
// group never ended) gives its ring slot back; nothing of it was queued.
struct PendingLaunch {
    std::unique_ptr<H2DLaunch> p;
    ~PendingLaunch()
    {
        if (p) release_slot(p->ring, p->slot, false);
    }
};

thread_local PendingLaunch t_pending;

// SECURE_INFER_VERIFY_BEFORE_RELEASE=1 (the counterpart of the reference's
// PIPE_GCM_DIRECT_VERIFIED_RELEASE switch, secure_infer.cpp:5528-5538): the
// host pipeline's reloads verify every tag before any plaintext reaches the
// cache (SI_RELOAD_VERIFY_BEFORE_RELEASE).
uint32_t reload_flags()
{
    static const uint32_t f = [] {
        const char* e = std::getenv("SECURE_INFER_VERIFY_BEFORE_RELEASE");
        return (e && std::atoi(e) != 0) ? uint32_t(SI_RELOAD_VERIFY_BEFORE_RELEASE) : 0u;
    }();
    return f;
}

// Largest pending launch in wire bytes (SECURE_INFER_H2D_BATCH_MB, default 64):
// ring slots are sized to the launches they carry.
uint64_t launch_byte_cap()
{
    static const uint64_t b = [] {
        uint64_t mb = 64;
        if (const char* e = std::getenv("SECURE_INFER_H2D_BATCH_MB")) mb = uint64_t(std::max(1, std::atoi(e)));
        return mb << 20;
    }();
    return b;
}

// A free slot of the ring, waited for if its previous launch is still
// running; nullptr if every slot is held by a launch not yet issued.
Mirror* claim_slot(StreamRing* ring, size_t& idx)
{
    std::lock_guard<std::mutex> g(ring->lock);
    for (size_t k = 0; k < ring->slots.size(); ++k) {
        const size_t i = ring->next;
        ring->next = (ring->next + 1) % ring->slots.size();
        if (ring->busy[i]) continue;
        Mirror& sl = *ring->slots[i];
        if (ring->used[i]) {
            if (hipEventSynchronize(sl.ev_b) != hipSuccess) return nullptr;
            profile_retire(sl);
            sl.held.clear();  // the copies from prefetch buffers are complete
            ring->used[i] = false;
        }
        ring->busy[i] = true;
        idx = i;
        return &sl;
    }
    return nullptr;
}

void release_slot(StreamRing* ring, size_t idx, bool launched)
{
    std::lock_guard<std::mutex> g(ring->lock);
    ring->busy[idx] = false;
    ring->used[idx] = launched;
}

// Issues the calling thread's pending launch: copies on the ring's copy
// stream, the caller's stream waits for them, then the fused reload.
int flush_launch()
{
    std::unique_ptr<H2DLaunch> L = std::move(t_pending.p);
    if (!L) return 0;
    if (L->n == 0) {  // its only swap failed before adding records
        release_slot(L->ring, L->slot, false);
        return 0;
    }
    Mirror& sl = *L->ring->slots[L->slot];
    const bool prof = profile_on();
    const size_t wire_cap = size_t(L->cap) * L->stride;
    // Device order: the K parts, then the V parts, each in swap order.
    std::vector<size_t> order;
    order.reserve(L->parts.size());
    for (uint32_t kind = 0; kind < 2; ++kind)
        for (size_t i = 0; i < L->parts.size(); ++i)
            if (L->parts[i].kind == kind) order.push_back(i);
    {
        uint32_t r = 0;
        for (size_t i : order) {
            L->parts[i].dev_r0 = r;
            r += L->parts[i].n;
        }
    }
    bool contiguous = true;  // tickets t0 .. t0 + n - 1 in device order
    for (size_t k = 1; k < order.size(); ++k)
        contiguous = contiguous && L->parts[order[k]].t0 == L->parts[order[k - 1]].t0 + L->parts[order[k - 1]].n;
    const size_t iv_bytes = contiguous ? 0 : size_t(L->n) * 16;
    uint8_t* tail = sl.host + wire_cap;
    if (!contiguous) {
        uint32_t* w = reinterpret_cast<uint32_t*>(tail);
        const uint32_t salt = (uint32_t(L->keys.salt[0]) << 24) | (uint32_t(L->keys.salt[1]) << 16) |
                              (uint32_t(L->keys.salt[2]) << 8) | uint32_t(L->keys.salt[3]);
        for (const H2DPart& p : L->parts)
            for (uint32_t r = 0; r < p.n; ++r) {
                const uint64_t c = L->keys.nonce + p.t0 + r;
                uint32_t* o = w + 4 * size_t(p.dev_r0 + r);
                o[0] = salt;
                o[1] = uint32_t(c >> 32);
                o[2] = uint32_t(c);
                o[3] = 2;
            }
    }
    int64_t* ids = reinterpret_cast<int64_t*>(tail + iv_bytes);
    for (const H2DPart& p : L->parts) memcpy(ids + p.dev_r0, L->slot_ids.data() + p.ids0, size_t(p.n) * 8);
    for (H2DPart& p : L->parts)
        if (p.ob) p.ob->status_off = p.dev_r0;  // the kernel stores statuses in device order

    bool launched = false;
    // On failure nothing is registered; copies still queued are waited for
    // before the prefetch buffers they read from are let go, and the status
    // buffer is never reused (the kernel may have been queued).
    auto fail = [&]() {
        if (L->status) L->status->orphaned = true;
        (void)hipStreamSynchronize(L->ring->copy);
        if (launched) (void)hipStreamSynchronize(L->stream);
        release_slot(L->ring, L->slot, false);
        return -1;
    };
    if (prof && hipEventRecord(sl.p_c0, L->ring->copy) != hipSuccess) return fail();
    const auto t_copy = std::chrono::steady_clock::now();
    // A launch of exactly one group prefetch (its K half, then its V half, as
    // large as the launch and with one ticket run), or of exactly one layer
    // prefetch: the prefetch buffer holds the records in device order
    // followed by the launch's tail (slot ids; a layer prefetch's IV words
    // first), so one copy carries all of it.
    const Prefetch* first = L->parts[order[0]].pf.get();
    bool one_copy = false;
    if (first && L->cap == L->n) {
        const Prefetch* owner = first->owner ? first->owner.get() : first;
        bool same_buffer = true;
        for (size_t i : order) {
            const Prefetch* pf = L->parts[i].pf.get();
            same_buffer = same_buffer && pf && (pf == owner || pf->owner.get() == owner) &&
                          L->parts[i].src == owner->host + size_t(L->parts[i].dev_r0) * L->stride;
        }
        if (same_buffer && owner->group_records == L->n && contiguous)
            one_copy = memcmp(owner->group_ids, ids, size_t(L->n) * 8) == 0;
        else if (same_buffer && owner->layer_records == L->n && !contiguous)
            one_copy = memcmp(owner->layer_tail, tail, iv_bytes + size_t(L->n) * 8) == 0;
    }
    if (one_copy) {
        if (hipMemcpyAsync(sl.dev, L->parts[order[0]].src, size_t(L->n) * L->stride + iv_bytes + size_t(L->n) * 8,
                           hipMemcpyHostToDevice, L->ring->copy) != hipSuccess)
            return fail();
    } else {
        // One copy per run of parts (in device order) whose sealed records sit
        // back to back, then the IV words and slot ids.
        for (size_t k = 0; k < order.size();) {
            const H2DPart& p0 = L->parts[order[k]];
            const uint8_t* src = p0.src;
            uint32_t rows = p0.n;
            size_t j = k + 1;
            for (; j < order.size() && L->parts[order[j]].src == src + size_t(rows) * L->stride; ++j)
                rows += L->parts[order[j]].n;
            if (hipMemcpyAsync(sl.dev + size_t(p0.dev_r0) * L->stride, src, size_t(rows) * L->stride,
                               hipMemcpyHostToDevice, L->ring->copy) != hipSuccess)
                return fail();
            k = j;
        }
        if (hipMemcpyAsync(sl.dev + wire_cap, tail, iv_bytes + size_t(L->n) * 8, hipMemcpyHostToDevice,
                           L->ring->copy) != hipSuccess)
            return fail();
    }
    const double copy_enqueue_us = us_since(t_copy);
    if ((prof && hipEventRecord(sl.p_c1, L->ring->copy) != hipSuccess) ||
        hipEventRecord(sl.ev_a, L->ring->copy) != hipSuccess || hipStreamWaitEvent(L->stream, sl.ev_a, 0) != hipSuccess)
        return fail();

    si_reload_desc d{};
    d.wire = sl.dev;
    d.wire_stride = L->stride;
    d.bytes = L->bytes;
    d.nrec = L->n;
    d.n_k = L->n_k;
    d.iv_words = contiguous ? nullptr : reinterpret_cast<const uint32_t*>(sl.dev + wire_cap);
    d.ticket_base = contiguous ? L->parts[order[0]].t0 : 0;
    d.cache_k = L->cache[0] ? L->cache[0] : L->cache[1];
    d.cache_v = L->cache[1] ? L->cache[1] : L->cache[0];
    d.slot_bytes = L->slot_bytes;
    d.nslots = L->nslots;
    d.slots = reinterpret_cast<const int64_t*>(sl.dev + wire_cap + iv_bytes);
    d.codec_bits = L->codec;
    d.heads = L->heads;
    d.head_dim = L->dim;
    d.layer = L->layer;
    d.staging = sl.stage;
    d.fail_count = L->fail_count;
    d.status_out = L->status ? L->status->dev : nullptr;
    d.flags = reload_flags();
    if (prof && hipEventRecord(sl.p_k0, L->stream) != hipSuccess) return fail();
    const auto t_kernel = std::chrono::steady_clock::now();
    if (secure_infer_gpu_reload_layer(L->stream, L->s, &d) != 0) return fail();
    const double kernel_enqueue_us = us_since(t_kernel);
    launched = true;
    if ((prof && hipEventRecord(sl.p_k1, L->stream) != hipSuccess) ||
        hipEventRecord(sl.ev_b, L->stream) != hipSuccess ||
        (L->status && hipEventRecord(L->status->ready, L->stream) != hipSuccess))
        return fail();
    for (H2DPart& p : L->parts)
        if (p.pf) sl.held.push_back(std::move(p.pf));
    if (prof) {
        sl.row.pending = true;
        sl.row.layer = L->layer;
        sl.row.kind = L->n_k == L->n ? 0u : (L->n_k == 0 ? 1u : 2u);
        sl.row.n = L->n;
        sl.row.bytes = L->bytes;
        sl.row.source = L->parts[0].source;
        sl.row.seal_us = 0;
        for (const H2DPart& p : L->parts) sl.row.seal_us += p.seal_us;
        sl.row.stride = L->stride;
        sl.row.copy_enqueue_us = copy_enqueue_us;
        sl.row.kernel_enqueue_us = kernel_enqueue_us;
        sl.row.rec_seal_us.clear();
        sl.row.rec_prefetched.clear();
        if (profile_records()) {
            for (size_t i : order) {
                const H2DPart& p = L->parts[i];
                for (uint32_t r = 0; r < p.n; ++r) {
                    sl.row.rec_seal_us.push_back(r < p.rec_us.size() ? p.rec_us[r] : 0.0f);
                    sl.row.rec_prefetched.push_back(p.source != 0 ? 1 : 0);
                }
            }
        }
    }
    release_slot(L->ring, L->slot, true);
    if (L->observe) {
        std::lock_guard<std::mutex> go(g_obs_lock);
        sweep_observed_locked();
        for (H2DPart& p : L->parts) g_observed.emplace(L->layer, std::move(p.ob));
    }
    return 0;
}

int h2d_swap_impl(hipStream_t stream, si_session* s, const void* host_base, uint64_t host_block_bytes,
                  uint64_t host_nblocks, void* dev_cache, uint64_t slot_bytes, uint64_t nslots,
                  const int64_t* mapping, uint32_t n, uint32_t kind, uint32_t layer, uint32_t codec_bits,
                  uint32_t heads, uint32_t head_dim, uint32_t* fail_count, bool observe, bool defer)
{
    if (!s || !host_base || !dev_cache || !mapping || n == 0 || kind > 1 || nslots == 0 || host_nblocks == 0)
        return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    if (!valid_mapping(mapping, n, true, host_nblocks, nslots)) return -1;
    const si_internal::SessionKeys keys = si_internal::session_keys(s);
    if (bytes > keys.max_record_bytes) return -1;
    DeviceState* ds = device_state();
    if (!ds) return -1;
    StreamRing* ring = ring_of(ds, stream);
    if (!ring) return -1;
    const uint64_t stride = secure_infer_wire_stride(bytes);
    const uint64_t tag_off = tag_offset(bytes);

    // Joins the pending launch if it takes these records, else issues that first.
    H2DLaunch* L = t_pending.p.get();
    if (L && !(L->stream == stream && L->s == s && L->ds == ds && L->layer == layer && L->codec == codec_bits &&
               L->heads == heads && L->dim == head_dim && L->bytes == bytes && L->slot_bytes == slot_bytes &&
               L->nslots == nslots && L->fail_count == fail_count && L->observe == observe &&
               (L->cache[kind] == nullptr || L->cache[kind] == dev_cache) && L->n + n <= L->cap)) {
        if (flush_launch() != 0) return -1;
        L = nullptr;
    }

    // Records sealed ahead of demand for exactly this swap, if any.
    std::shared_ptr<Prefetch> pf = take_prefetch(s, host_base, host_block_bytes, mapping, n, kind, layer, codec_bits);
    uint32_t source = 0;
    if (pf) {
        std::unique_lock<std::mutex> g(pf->m);
        source = pf->done == pf->tasks ? 1u : 2u;
        pf->cv.wait(g, [&] { return pf->done == pf->tasks; });
        if (pf->failed) return -1;
        (source == 1 ? g_pf_ready : g_pf_waited).fetch_add(1);
    } else {
        g_pf_missing.fetch_add(1);
    }

    if (!L) {
        auto nl = std::make_unique<H2DLaunch>();
        uint64_t cap = n;
        if (defer) {
            const int64_t expected = si_internal::group_expected();
            const uint64_t fit = std::max<uint64_t>(1, launch_byte_cap() / stride);
            cap = std::max<uint64_t>(n, std::min<uint64_t>(expected > 0 ? uint64_t(expected) : 0, fit));
        }
        nl->cap = uint32_t(std::min<uint64_t>(cap, UINT32_MAX / 2));
        if (nl->cap < n) return -1;
        Mirror* sl = claim_slot(ring, nl->slot);
        if (!sl) return -1;
        nl->ring = ring;
        if (!sl->reserve(size_t(nl->cap) * (stride + 24), codec_bits ? size_t(nl->cap) * tag_off : 0) ||
            (profile_on() && !sl->init_profile())) {
            release_slot(ring, nl->slot, false);
            return -1;
        }
        if (observe && !(nl->status = share_status(ds, take_status(ds, nl->cap)))) {
            release_slot(ring, nl->slot, false);
            return -1;
        }
        nl->stream = stream;
        nl->s = s;
        nl->hold.take(s);
        nl->keys = keys;
        nl->ds = ds;
        nl->layer = layer;
        nl->codec = codec_bits;
        nl->heads = heads;
        nl->dim = head_dim;
        nl->bytes = bytes;
        nl->stride = stride;
        nl->tag_off = tag_off;
        nl->slot_bytes = slot_bytes;
        nl->nslots = nslots;
        nl->fail_count = fail_count;
        nl->observe = observe;
        t_pending.p = std::move(nl);
        L = t_pending.p.get();
    }

    // Host side: seal on demand into the slot's rows, or take the prefetched records.
    Mirror& sl = *ring->slots[L->slot];
    H2DPart part;
    part.r0 = L->n;
    part.n = n;
    part.kind = kind;
    part.ids0 = L->slot_ids.size();
    part.source = source;
    const bool prof_records = profile_records();
    if (pf) {
        part.src = pf->host;
        part.t0 = pf->t0;
        part.seal_us = pf->seal_us;
        if (prof_records) part.rec_us = pf->rec_us;
        part.pf = pf;
    } else {
        const auto ts = std::chrono::steady_clock::now();
        part.t0 = si_internal::reserve_tickets(n);
        if (!si_internal::replay_reserve_range(part.t0, n)) {
            fprintf(stderr, "[secure_infer] duplicate H2D transfer tickets rejected at %llu\n",
                    static_cast<unsigned long long>(part.t0));
            return -1;
        }
        uint8_t* rows = sl.host + size_t(part.r0) * stride;
        const uint64_t t0 = part.t0;
        std::atomic<int> bad{0};
        if (prof_records) part.rec_us.assign(n, 0.0f);
        Pool::get().parallel_for(n, [&](size_t r) {
            const int64_t hb = mapping[2 * r];
            bool ok = true;
            const auto tr = std::chrono::steady_clock::now();
            seal_record(keys, static_cast<const uint8_t*>(host_base) + uint64_t(hb) * host_block_bytes, bytes,
                        tag_off, t0 + r, rows + r * stride, layer, kind, hb, ok);
            if (prof_records) part.rec_us[r] = float(us_since(tr));
            if (!ok) bad.store(1);
        });
        if (bad.load()) return -1;
        part.src = rows;
        part.seal_us = us_since(ts);
    }
    if (observe) {
        auto ob = std::make_shared<Observed>();
        ob->ds = ds;
        ob->session = s;
        ob->host_base = static_cast<const uint8_t*>(host_base);
        ob->host_block_bytes = host_block_bytes;
        ob->host_nblocks = host_nblocks;
        ob->dev_cache = dev_cache;
        ob->slot_bytes = slot_bytes;
        ob->nslots = nslots;
        ob->kind = kind;
        ob->layer = layer;
        ob->codec = codec_bits;
        ob->heads = heads;
        ob->dim = head_dim;
        ob->stream = stream;
        ob->job_id = si_internal::current_job_id();
        ob->mapping.assign(mapping, mapping + 2 * size_t(n));
        ob->status = L->status;
        ob->status_off = part.r0;
        part.ob = std::move(ob);
    }
    for (uint32_t r = 0; r < n; ++r) L->slot_ids.push_back(mapping[2 * r + 1]);
    L->cache[kind] = dev_cache;
    L->n += n;
    if (kind == 0) L->n_k += n;
    L->parts.push_back(std::move(part));
    return defer ? 0 : flush_launch();
}

// ---------------------------------------------------------------- D2H batches

struct D2HBatch;

// One record of a D2H launch: where it authenticates into and its ticket.
struct D2HRec {
    uint8_t* dst = nullptr;
    uint64_t ticket = 0;
};

// The records of consecutive D2H swaps of one batch that are gathered,
// sealed and copied back as one launch: K swaps before V swaps, all of one
// stream, session, layer and geometry.  The buffer is laid out
// [n wire records][iv words, n x 16, only when the tickets are not one run]
// [slot ids, n x 8][device fail word, 16].
struct D2HJob {
    D2HBatch* batch = nullptr;
    DeviceState* ds = nullptr;
    std::unique_ptr<Mirror> buf;
    hipStream_t stream = nullptr;
    si_session* s = nullptr;
    si_internal::SessionHold hold;  // until the job is issued (or dropped)
    si_internal::SessionKeys keys{};
    uint32_t layer = 0, codec = 0, heads = 0, dim = 0;
    uint64_t bytes = 0, stride = 0, tag_off = 0, slot_bytes = 0, nslots = 0;
    const void* cache[2] = {nullptr, nullptr};
    uint32_t n = 0, n_k = 0;
    std::vector<D2HRec> recs;
    std::vector<int64_t> slot_ids;
    std::vector<uint8_t> aads;  // n x 64, copied into the records' AAD slots at issue
    uint64_t fail_off = 0;      // device u32 counting records with a bad slot id
    size_t counted = 0;         // buffer bytes counted in flight for the device
    size_t tasks_left = 0;      // verification tasks not finished (guarded by the batch's lock)
};

struct D2HBatch {
    DeviceState* ds = nullptr;
    uint64_t expected = 0;  // records the batch announced (batch_begin)
    bool group_open = false;
    std::vector<std::unique_ptr<D2HJob>> jobs;  // issued launches
    std::unique_ptr<D2HJob> pending;           // launch still taking swaps
    std::vector<hipStream_t> streams;
    std::vector<hipEvent_t> joins;
    std::mutex m;
    std::condition_variable cv;
    size_t pending_tasks = 0;  // verification tasks in flight (guarded by m)
    std::atomic<uint64_t> failures{0};

    // Waits until no worker touches the batch (its issued launches are
    // verified) and its device joins are done.
    void wait_done()
    {
        {
            std::unique_lock<std::mutex> g(m);
            cv.wait(g, [&] { return pending_tasks == 0; });
        }
        for (hipEvent_t e : joins) {
            (void)hipEventSynchronize(e);
            (void)hipEventDestroy(e);
        }
        joins.clear();
    }
    // A thread that ends inside a batch (no batch_end) still lets its issued
    // launches finish before the batch goes; the launch not yet issued is
    // dropped.
    ~D2HBatch() { wait_done(); }
};

thread_local std::unique_ptr<D2HBatch> t_batch;

// D2H launches a device keeps in flight: at most 6, and at most
// SECURE_INFER_D2H_INFLIGHT_MB (default 128) of buffers; an issue waits for
// earlier launches' verification beyond either.  Three or four in flight keep
// the copy engine and the verifiers busy.  More only queue copies: with ten
// 42-MB copies queued, enqueueing the next one blocked the issuing thread for
// ~12 ms (MI355X, ROCm 7.2), and the GPU's queue ran dry meanwhile.
constexpr size_t kD2HMaxJobs = 6;

// Largest D2H launch in wire bytes (SECURE_INFER_D2H_LAUNCH_MB, default 64):
// a batch's swaps of one layer merge into launches up to this size.  A store
// job's batch spans every layer, so one layer's host authentication overlaps
// the next layer's copy; smaller launches measured slower there (70B int4
// layer, 42 MB: 8 MB launches 1480 us per layer, 64 MB 830 us).
uint64_t d2h_launch_cap()
{
    static const uint64_t b = [] {
        uint64_t mb = 64;
        if (const char* e = std::getenv("SECURE_INFER_D2H_LAUNCH_MB")) mb = uint64_t(std::max(1, std::atoi(e)));
        return mb << 20;
    }();
    return b;
}

size_t d2h_inflight_budget()
{
    static const size_t b = [] {
        size_t mb = 128;
        if (const char* e = std::getenv("SECURE_INFER_D2H_INFLIGHT_MB")) mb = size_t(std::max(1, std::atoi(e)));
        return mb << 20;
    }();
    return b;
}

// A D2H buffer of at least `need` bytes (and `stage` bytes of codec staging),
// counted in flight until put_buffer.
std::unique_ptr<Mirror> take_buffer(DeviceState* ds, size_t need, size_t stage)
{
    std::unique_ptr<Mirror> b;
    {
        std::unique_lock<std::mutex> g(ds->pool_lock);
        ds->d2h_cv.wait(g, [&] {
            return ds->d2h_jobs == 0 ||
                   (ds->d2h_jobs < kD2HMaxJobs && ds->d2h_inflight + need <= d2h_inflight_budget());
        });
        ds->d2h_inflight += need;
        ++ds->d2h_jobs;
        size_t best = ds->free_bufs.size();
        for (size_t i = 0; i < ds->free_bufs.size(); ++i)
            if (ds->free_bufs[i]->cap >= need &&
                (best == ds->free_bufs.size() || ds->free_bufs[i]->cap < ds->free_bufs[best]->cap))
                best = i;
        if (best == ds->free_bufs.size() && !ds->free_bufs.empty()) best = ds->free_bufs.size() - 1;
        if (best < ds->free_bufs.size()) {
            b = std::move(ds->free_bufs[best]);
            ds->free_bufs.erase(ds->free_bufs.begin() + long(best));
        }
    }
    if (!b) {
        b = std::make_unique<Mirror>();
        if (!b->init()) b.reset();
    }
    if (!b || !b->reserve(need, stage)) {
        std::lock_guard<std::mutex> g(ds->pool_lock);
        ds->d2h_inflight -= need;
        --ds->d2h_jobs;
        ds->d2h_cv.notify_all();
        return nullptr;
    }
    return b;
}

void put_buffer(DeviceState* ds, std::unique_ptr<Mirror> b, size_t counted)
{
    std::lock_guard<std::mutex> g(ds->pool_lock);
    ds->d2h_inflight -= counted;
    --ds->d2h_jobs;
    if (b) ds->free_bufs.push_back(std::move(b));
    ds->d2h_cv.notify_all();
}

// A batch that announced no more than a few launches' worth of records (one
// layer stored on its own) is cut into about four launches, so that its
// copies and host authentication still overlap (70B int4 layer alone:
// 1.8 ms with one launch, 1.35 ms with four); a batch of many layers keeps
// whole-layer launches, which overlap across layers.
uint64_t d2h_batch_launch_cap(const D2HBatch& b, uint64_t stride)
{
    const uint64_t cap = d2h_launch_cap();
    if (b.expected == 0) return cap;
    const uint64_t quarter = b.expected * stride / 4;
    return std::min(cap, std::max<uint64_t>(uint64_t(8) << 20, quarter));
}

size_t job_bytes(const D2HJob& j, bool ivs) { return size_t(j.n) * (j.stride + (ivs ? 24 : 8)) + 16; }

// SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE=1: a D2H record that fails host
// authentication zeroes its host block and then aborts the process, as the
// reference does (secure_infer.cpp:2514-2524, 8550-8555); by default the
// batch fails instead (batch_end returns -1) and the process goes on.
bool d2h_abort_on_failure()
{
    static const bool a = [] {
        const char* e = std::getenv("SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE");
        return e && std::atoi(e) != 0;
    }();
    return a;
}

void verify_records(D2HJob* job, uint32_t r0, uint32_t r1)
{
    D2HBatch* b = job->batch;
    uint64_t bad = 0;
    if (hipEventSynchronize(job->buf->ev_b) != hipSuccess) {
        bad = r1 - r0;
    } else {
        // The device's count of records sealed over a bad slot id (checked by
        // the first task of the job; such a record also carries a tag that
        // cannot verify).
        if (r0 == 0) {
            uint32_t dev_fail = 0;
            memcpy(&dev_fail, job->buf->host + job->fail_off, 4);
            bad += dev_fail;
        }
        for (uint32_t r = r0; r < r1; ++r) {
            uint8_t* rec = job->buf->host + uint64_t(r) * job->stride;
            uint8_t* dst = job->recs[r].dst;
            if (take_shot(g_tamper_d2h)) rec[0] ^= 0x01;
            uint8_t iv[12];
            record_iv(job->keys, job->recs[r].ticket, iv);
            if (!gcm_open(job->keys.key, iv, rec + job->tag_off + 32, 64, rec, job->bytes,
                          rec + job->tag_off, dst)) {
                memset(dst, 0, job->bytes);  // fail closed
                ++bad;
            }
        }
    }
    if (bad) b->failures.fetch_add(bad);
    if (bad && d2h_abort_on_failure()) {
        fprintf(stderr,
                "[secure_infer] D2H authentication failed: %llu record(s) withheld (host blocks zeroed); "
                "aborting (SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE)\n",
                static_cast<unsigned long long>(bad));
        std::abort();
    }
    // The decrements and the notification happen under the batch's lock:
    // batch_end may destroy the batch as soon as it sees pending_tasks == 0.
    // The job's buffer goes back to the device's pool after its last task.
    std::unique_ptr<Mirror> done;
    bool last = false;
    {
        std::lock_guard<std::mutex> g(b->m);
        if (--job->tasks_left == 0) {
            done = std::move(job->buf);
            last = true;
        }
    }
    if (last) put_buffer(job->ds, std::move(done), job->counted);
    std::lock_guard<std::mutex> g(b->m);
    if (--b->pending_tasks == 0) b->cv.notify_all();
}

// Hands a launch's records to the worker pool once its copies are done.
void d2h_copied(D2HJob* job)
{
    const uint32_t per_task = 4;
    std::vector<std::function<void()>> tasks;
    for (uint32_t r0 = 0; r0 < job->n; r0 += per_task) {
        const uint32_t r1 = std::min(job->n, r0 + per_task);
        tasks.emplace_back([job, r0, r1] { verify_records(job, r0, r1); });
    }
    Pool::get().submit_all(tasks);
}

// One thread per device waits for issued launches' copies in issue order
// (the order the D2H stream runs them) and hands each to the worker pool
// -- the reference's host callback after a group's copy
// (d2h_group_ready_callback via aclrtLaunchHostFunc, secure_infer.cpp:2880-2895).
// A host function on the D2H stream itself would hold the stream until the
// runtime's callback thread has run it, a gap after every launch's copy.
struct D2HWatcher {
    std::mutex m;
    std::condition_variable cv;
    std::deque<D2HJob*> q;
};

void d2h_watch(DeviceState* ds, D2HJob* job)
{
    D2HWatcher& w = *ds->watcher;
    {
        std::lock_guard<std::mutex> g(w.m);
        w.q.push_back(job);
    }
    w.cv.notify_one();
}

bool start_watcher(DeviceState* ds)
{
    std::lock_guard<std::mutex> g(ds->pool_lock);
    if (ds->watcher) return true;
    ds->watcher = new D2HWatcher();  // never destroyed, like the worker pool
    D2HWatcher* w = ds->watcher;
    const int device = ds->device;
    std::thread([w, device] {
        (void)hipSetDevice(device);
        for (;;) {
            D2HJob* job = nullptr;
            {
                std::unique_lock<std::mutex> g(w->m);
                w->cv.wait(g, [&] { return !w->q.empty(); });
                job = w->q.front();
                w->q.pop_front();
            }
            (void)hipEventSynchronize(job->buf->ev_b);  // the tasks check the status again
            d2h_copied(job);
        }
    }).detach();
    return true;
}

// Issues the batch's pending launch: AADs, iv words, slot ids and a zeroed
// fail word up on the caller's stream, gather (+ quantise) + seal, then the
// records and the fail word down on the D2H stream, whose host function
// queues their authentication.
int d2h_issue(D2HBatch* b)
{
    std::unique_ptr<D2HJob> job = std::move(b->pending);
    if (!job || job->n == 0) return 0;
    if (!start_watcher(job->ds)) return -1;
    bool run = true;  // tickets t0 .. t0 + n - 1 in record order
    for (uint32_t r = 1; r < job->n; ++r) run = run && job->recs[r].ticket == job->recs[r - 1].ticket + 1;
    const size_t wire = size_t(job->n) * job->stride;
    const size_t iv_bytes = run ? 0 : size_t(job->n) * 16;
    job->fail_off = wire + iv_bytes + size_t(job->n) * 8;
    const size_t need = job_bytes(*job, !run);
    job->buf = take_buffer(job->ds, need, job->codec ? size_t(job->n) * job->tag_off : 0);
    if (!job->buf) return -1;
    job->counted = need;
    DeviceState* ds = job->ds;
    // On failure the buffer goes back to the pool once nothing queued uses it.
    auto fail = [&]() {
        (void)hipStreamSynchronize(job->stream);
        (void)hipStreamSynchronize(ds->d2h);
        put_buffer(ds, std::move(job->buf), job->counted);
        return -1;
    };
    uint8_t* h = job->buf->host;
    uint8_t* d = job->buf->dev;
    for (uint32_t r = 0; r < job->n; ++r) memcpy(h + size_t(r) * job->stride + job->tag_off + 32, &job->aads[64 * size_t(r)], 64);
    if (!run) {
        uint32_t* w = reinterpret_cast<uint32_t*>(h + wire);
        const uint32_t salt = (uint32_t(job->keys.salt[0]) << 24) | (uint32_t(job->keys.salt[1]) << 16) |
                              (uint32_t(job->keys.salt[2]) << 8) | uint32_t(job->keys.salt[3]);
        for (uint32_t r = 0; r < job->n; ++r) {
            const uint64_t c = job->keys.nonce + job->recs[r].ticket;
            w[4 * r] = salt;
            w[4 * r + 1] = uint32_t(c >> 32);
            w[4 * r + 2] = uint32_t(c);
            w[4 * r + 3] = 2;
        }
    }
    memcpy(h + wire + iv_bytes, job->slot_ids.data(), size_t(job->n) * 8);
    memset(h + job->fail_off, 0, 16);
    job->aads.clear();
    job->aads.shrink_to_fit();
    if (hipMemcpy2DAsync(d + job->tag_off + 32, job->stride, h + job->tag_off + 32, job->stride, 64, job->n,
                         hipMemcpyHostToDevice, job->stream) != hipSuccess ||
        hipMemcpyAsync(d + wire, h + wire, need - wire, hipMemcpyHostToDevice, job->stream) != hipSuccess)
        return fail();
    si_writeback_desc w{};
    w.wire = d;
    w.wire_stride = job->stride;
    w.bytes = job->bytes;
    w.nrec = job->n;
    w.n_k = job->n_k;
    w.iv_words = run ? nullptr : reinterpret_cast<const uint32_t*>(d + wire);
    w.ticket_base = run ? job->recs[0].ticket : 0;
    w.cache_k = const_cast<void*>(job->cache[0] ? job->cache[0] : job->cache[1]);
    w.cache_v = const_cast<void*>(job->cache[1] ? job->cache[1] : job->cache[0]);
    w.slot_bytes = job->slot_bytes;
    w.nslots = job->nslots;
    w.slots = reinterpret_cast<const int64_t*>(d + wire + iv_bytes);
    w.codec_bits = job->codec;
    w.heads = job->heads;
    w.head_dim = job->dim;
    w.layer = job->layer;
    w.staging = job->buf->stage;
    w.fail_count = reinterpret_cast<uint32_t*>(d + job->fail_off);
    if (secure_infer_gpu_writeback_layer(job->stream, job->s, &w) != 0) return fail();
    job->hold.reset();  // the session is not used past the launch
    if (hipEventRecord(job->buf->ev_a, job->stream) != hipSuccess ||
        hipStreamWaitEvent(ds->d2h, job->buf->ev_a, 0) != hipSuccess ||
        hipMemcpyAsync(h, d, wire, hipMemcpyDeviceToHost, ds->d2h) != hipSuccess ||
        hipMemcpyAsync(h + job->fail_off, d + job->fail_off, 16, hipMemcpyDeviceToHost, ds->d2h) != hipSuccess ||
        hipEventRecord(job->buf->ev_b, ds->d2h) != hipSuccess)
        return fail();
    job->tasks_left = (job->n + 3) / 4;
    {
        std::lock_guard<std::mutex> g(b->m);
        b->pending_tasks += job->tasks_left;
    }
    if (std::find(b->streams.begin(), b->streams.end(), job->stream) == b->streams.end())
        b->streams.push_back(job->stream);
    D2HJob* jp = job.get();
    b->jobs.push_back(std::move(job));
    d2h_watch(ds, jp);
    return 0;
}

}  // namespace

namespace si_internal {

int flush_pending_h2d() { return flush_launch(); }

int wait_observed_layer(uint32_t layer, bool* found)
{
    *found = false;
    if (flush_launch() != 0) return -1;
    for (unsigned round = 0;; ++round) {
        std::vector<std::shared_ptr<Observed>> recs;
        {
            std::lock_guard<std::mutex> g(g_obs_lock);
            auto range = g_observed.equal_range(layer);
            for (auto it = range.first; it != range.second; ++it) recs.push_back(it->second);
            g_observed.erase(range.first, range.second);
        }
        if (recs.empty()) return 0;
        *found = true;
        int rc = 0;
        // Records that failed once: (swap, index).
        std::vector<std::pair<Observed*, uint32_t>> retry;
        for (const auto& ob : recs) {
            const uint32_t n = uint32_t(ob->mapping.size() / 2);
            if (hipEventSynchronize(ob->status->ready) != hipSuccess) {
                rc = -1;
                continue;
            }
            for (uint32_t r = 0; r < n; ++r) {
                const uint32_t st = ob->status_of(r);
                if (st == 1u) continue;
                // A destroyed session (forget_session) cannot re-seal.
                if (st != 0u || round != 0 || !ob->session) rc = -1;
                else retry.emplace_back(ob.get(), r);
            }
        }
        if (rc == 0) {
            // A record that failed is re-sealed from the trusted host copy
            // under a fresh ticket; its verifier result is checked in the next
            // round, before the layer is used (secure_infer.cpp:7316-7330).
            for (size_t i = 0; i < retry.size() && rc == 0;) {
                Observed* ob = retry[i].first;
                std::vector<int64_t> part;
                for (; i < retry.size() && retry[i].first == ob; ++i) {
                    part.push_back(ob->mapping[2 * retry[i].second]);
                    part.push_back(ob->mapping[2 * retry[i].second + 1]);
                }
                const uint32_t m = uint32_t(part.size() / 2);
                // The retry runs on the device (and ring) the swap used.
                int cur = 0;
                if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(ob->ds->device) != hipSuccess) {
                    rc = -1;
                    break;
                }
                if (h2d_swap_impl(ob->stream, ob->session, ob->host_base, ob->host_block_bytes,
                                  ob->host_nblocks, ob->dev_cache, ob->slot_bytes, ob->nslots, part.data(), m,
                                  ob->kind, ob->layer, ob->codec, ob->heads, ob->dim, nullptr, true, false) != 0 ||
                    hipStreamSynchronize(ob->stream) != hipSuccess)
                    rc = -1;
                (void)hipSetDevice(cur);
            }
        }
        recs.clear();
        if (rc != 0) {
            // Drop the retries' own observations too: the layer has failed.
            std::lock_guard<std::mutex> g(g_obs_lock);
            auto range = g_observed.equal_range(layer);
            std::vector<std::shared_ptr<Observed>> rest;
            for (auto it = range.first; it != range.second; ++it) rest.push_back(it->second);
            g_observed.erase(range.first, range.second);
            for (auto& ob : rest) (void)hipEventSynchronize(ob->status->ready);
            return -1;
        }
        if (retry.empty()) return 0;
    }
}

bool forget_session(si_session* s)
{
    // The calling thread's pending launches may name the session: issue them.
    (void)flush_launch();
    if (D2HBatch* b = t_batch.get())
        if (b->pending && b->pending->s == s) (void)d2h_issue(b);
    if (session_holds(s) != 0) return false;
    std::vector<std::shared_ptr<Prefetch>> drop;
    {
        std::lock_guard<std::mutex> g(g_pf_lock);
        for (auto it = g_prefetch.begin(); it != g_prefetch.end();) {
            if ((*it)->session == s) {
                drop.push_back(std::move(*it));
                it = g_prefetch.erase(it);
            } else {
                ++it;
            }
        }
    }
    for (auto& pf : drop) wait_sealed(*pf);
    std::lock_guard<std::mutex> g(g_obs_lock);
    for (auto& e : g_observed)
        if (e.second->session == s) e.second->session = nullptr;
    return true;
}

int wait_observed_job(uint64_t job_id, bool* found)
{
    if (flush_launch() != 0) return 0;
    std::vector<std::shared_ptr<Observed>> recs;
    {
        std::lock_guard<std::mutex> g(g_obs_lock);
        for (auto it = g_observed.begin(); it != g_observed.end();) {
            if (it->second->job_id == job_id) {
                recs.push_back(it->second);
                it = g_observed.erase(it);
            } else {
                ++it;
            }
        }
    }
    if (recs.empty()) return 1;
    *found = true;
    bool valid = true;
    for (auto& ob : recs) {
        const uint32_t n = uint32_t(ob->mapping.size() / 2);
        if (hipEventSynchronize(ob->status->ready) != hipSuccess) {
            valid = false;
        } else {
            for (uint32_t r = 0; r < n; ++r) valid = valid && ob->status_of(r) == 1u;
        }
    }
    return valid ? 1 : 0;
}

}  // namespace si_internal

extern "C" {

int secure_infer_host_threads(void) { return int(Pool::get().threads()); }

int secure_infer_h2d_swap(hipStream_t stream, si_session* s, const void* host_base,
                          uint64_t host_block_bytes, uint64_t host_nblocks, void* dev_cache,
                          uint64_t slot_bytes, uint64_t nslots, const int64_t* mapping, uint32_t n,
                          uint32_t kind, uint32_t layer, uint32_t codec_bits, uint32_t heads,
                          uint32_t head_dim, uint32_t* fail_count)
{
    // Every swap is observed, inside a layer group or not, as the reference
    // observes its unbatched copies too (secure_infer.cpp:7036-7052): a
    // failed record reaches wait_layer_authentication whether or not the
    // caller passed a fail counter.
    return h2d_swap_impl(stream, s, host_base, host_block_bytes, host_nblocks, dev_cache, slot_bytes, nslots,
                         mapping, n, kind, layer, codec_bits, heads, head_dim, fail_count, true,
                         si_internal::group_open());
}

int secure_infer_h2d_prefetch(si_session* s, const void* host_base, uint64_t host_block_bytes, uint64_t host_nblocks,
                              const int64_t* mapping, uint32_t n, uint32_t kind, uint32_t layer, uint32_t codec_bits,
                              uint32_t heads, uint32_t head_dim)
{
    if (!s || !host_base || !mapping || n == 0 || kind > 1 || host_nblocks == 0) return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    for (uint32_t r = 0; r < n; ++r)
        if (mapping[2 * r] < 0 || uint64_t(mapping[2 * r]) >= host_nblocks) return -1;
    const si_internal::SessionKeys keys = si_internal::session_keys(s);
    if (bytes > keys.max_record_bytes) return -1;
    const uint64_t stride = secure_infer_wire_stride(bytes);
    size_t cap = 0;
    uint8_t* buf = take_pf_buffer(size_t(n) * stride, cap);
    if (!buf) return -1;  // over SECURE_INFER_PREFETCH_MB: the swap seals on demand
    auto pf = new_prefetch(s, keys, host_base, host_block_bytes, mapping, n, kind, layer, codec_bits, heads,
                           head_dim, bytes, buf);
    pf->cap = cap;
    pf->t0 = si_internal::reserve_tickets(n);
    if (!si_internal::replay_reserve_range(pf->t0, n)) return -1;
    std::vector<std::function<void()>> tasks;
    queue_seals(pf, tasks);
    Pool::get().submit_all(tasks);
    return 0;
}

int secure_infer_h2d_prefetch_group(si_session* s, const void* k_base, const void* v_base,
                                    uint64_t host_block_bytes, uint64_t host_nblocks, const int64_t* mapping,
                                    uint32_t n, uint32_t layer, uint32_t codec_bits, uint32_t heads,
                                    uint32_t head_dim)
{
    if (!s || !k_base || !v_base || !mapping || n == 0 || host_nblocks == 0 || n > UINT32_MAX / 2) return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    for (uint32_t r = 0; r < n; ++r)
        if (mapping[2 * r] < 0 || uint64_t(mapping[2 * r]) >= host_nblocks) return -1;
    const si_internal::SessionKeys keys = si_internal::session_keys(s);
    if (bytes > keys.max_record_bytes) return -1;
    const uint64_t stride = secure_infer_wire_stride(bytes);
    const size_t wire = size_t(2) * n * stride;
    size_t cap = 0;
    uint8_t* buf = take_pf_buffer(wire + size_t(2) * n * 8, cap);
    if (!buf) return -1;
    // The slot ids of both halves after the records: the device layout of a
    // launch of exactly this group ([2n records][2n slot ids]).
    for (uint32_t h = 0; h < 2; ++h)
        for (uint32_t r = 0; r < n; ++r) memcpy(buf + wire + (size_t(h) * n + r) * 8, &mapping[2 * r + 1], 8);
    auto pk = new_prefetch(s, keys, k_base, host_block_bytes, mapping, n, 0, layer, codec_bits, heads, head_dim,
                           bytes, buf);
    pk->cap = cap;
    pk->group_ids = buf + wire;
    pk->group_records = 2 * n;
    auto pv = new_prefetch(s, keys, v_base, host_block_bytes, mapping, n, 1, layer, codec_bits, heads, head_dim,
                           bytes, buf + size_t(n) * stride);
    pv->owner = pk;
    // K then V: the tickets a group's two swaps take in that order.
    pk->t0 = si_internal::reserve_tickets(2 * n);
    pv->t0 = pk->t0 + n;
    if (!si_internal::replay_reserve_range(pk->t0, 2 * uint64_t(n))) return -1;
    std::vector<std::function<void()>> tasks;
    queue_seals(pk, tasks);
    queue_seals(pv, tasks);
    Pool::get().submit_all(tasks);
    return 0;
}

int secure_infer_h2d_prefetch_layer(si_session* s, const void* k_base, const void* v_base, uint64_t host_block_bytes,
                                    uint64_t host_nblocks, const int64_t* mapping, const uint32_t* group_start,
                                    const uint32_t* group_rows, uint32_t ngroups, uint32_t layer, uint32_t codec_bits,
                                    uint32_t heads, uint32_t head_dim)
{
    if (!s || !k_base || !v_base || !mapping || !group_start || !group_rows || ngroups == 0 || host_nblocks == 0)
        return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    uint64_t total = 0;
    for (uint32_t g = 0; g < ngroups; ++g) {
        if (group_rows[g] == 0) return -1;
        for (uint32_t r = 0; r < group_rows[g]; ++r) {
            const int64_t hb = mapping[2 * (uint64_t(group_start[g]) + r)];
            if (hb < 0 || uint64_t(hb) >= host_nblocks) return -1;
        }
        total += group_rows[g];
    }
    if (total > UINT32_MAX / 4) return -1;
    const uint32_t N = uint32_t(total);
    const si_internal::SessionKeys keys = si_internal::session_keys(s);
    if (bytes > keys.max_record_bytes) return -1;
    const uint64_t stride = secure_infer_wire_stride(bytes);
    const size_t wire = size_t(2) * N * stride;
    size_t cap = 0;
    uint8_t* buf = take_pf_buffer(wire + size_t(2) * N * (16 + 8), cap);
    if (!buf) return -1;
    // Tickets in the order the swaps take them (each group's K, then its V):
    // the records keep the reference's tickets while the buffer holds every K
    // record before every V record, with explicit IV words.
    const uint64_t t0 = si_internal::reserve_tickets(2 * N);
    uint32_t* ivw = reinterpret_cast<uint32_t*>(buf + wire);
    int64_t* ids = reinterpret_cast<int64_t*>(buf + wire + size_t(2) * N * 16);
    const uint32_t salt = (uint32_t(keys.salt[0]) << 24) | (uint32_t(keys.salt[1]) << 16) |
                          (uint32_t(keys.salt[2]) << 8) | uint32_t(keys.salt[3]);
    std::vector<std::shared_ptr<Prefetch>> parts;
    uint32_t off = 0;  // K rows of the groups before this one
    for (uint32_t g = 0; g < ngroups; ++g) {
        const uint32_t n = group_rows[g];
        const int64_t* map = mapping + 2 * uint64_t(group_start[g]);
        for (uint32_t kind = 0; kind < 2; ++kind) {
            const uint32_t row = kind * N + off;  // device row of the part's first record
            auto pf = new_prefetch(s, keys, kind ? v_base : k_base, host_block_bytes, map, n, kind, layer, codec_bits,
                                   heads, head_dim, bytes, buf + size_t(row) * stride);
            pf->t0 = t0 + 2 * uint64_t(off) + uint64_t(kind) * n;
            for (uint32_t r = 0; r < n; ++r) {
                const uint64_t c = keys.nonce + pf->t0 + r;
                uint32_t* o = ivw + 4 * size_t(row + r);
                o[0] = salt;
                o[1] = uint32_t(c >> 32);
                o[2] = uint32_t(c);
                o[3] = 2;
                ids[row + r] = map[2 * r + 1];
            }
            if (parts.empty()) {
                pf->cap = cap;
                pf->layer_tail = buf + wire;
                pf->layer_records = 2 * N;
            } else {
                pf->owner = parts.front();
            }
            parts.push_back(std::move(pf));
        }
        off += n;
    }
    // (On failure the parts go, and the first returns the buffer to the pool.)
    if (!si_internal::replay_reserve_range(t0, 2 * uint64_t(N))) return -1;
    std::vector<std::function<void()>> tasks;
    for (auto& pf : parts) queue_seals(pf, tasks);
    Pool::get().submit_all(tasks);
    return 0;
}

void secure_infer_get_transfer_prefetch_stats(uint64_t* ready, uint64_t* busy_fallback, uint64_t* missing_fallback)
{
    if (ready) *ready = g_pf_ready.load();
    if (busy_fallback) *busy_fallback = g_pf_waited.load();
    if (missing_fallback) *missing_fallback = g_pf_missing.load();
}

uint64_t secure_infer_count_ready_unconsumed_gcm_tickets(void)
{
    uint64_t n = 0;
    std::lock_guard<std::mutex> g(g_pf_lock);
    for (const auto& pf : g_prefetch) {
        std::lock_guard<std::mutex> gp(pf->m);
        if (pf->done == pf->tasks && !pf->failed) n += pf->n;
    }
    return n;
}

void secure_infer_retire_transfer_prefetches(void)
{
    std::vector<std::shared_ptr<Prefetch>> drop;
    {
        std::lock_guard<std::mutex> g(g_pf_lock);
        drop.swap(g_prefetch);
    }
    // Sealing tasks still running hold their prefetch; its buffer returns to
    // the free list when the last holder lets go.  Their tickets stay used.
    for (auto& pf : drop) wait_sealed(*pf);
}

void secure_infer_invalidate_transfer_prefetches(void) { secure_infer_retire_transfer_prefetches(); }

void secure_infer_flush_completed_h2d_profile(void) { profile_sweep(false); }

void secure_infer_drain_h2d_profile_after_job(void) { profile_sweep(true); }

void secure_infer_pause_h2d_profile(int paused) { g_profile_paused.store(paused != 0); }

int secure_infer_test_tamper_h2d(int32_t layer, int32_t kind, int64_t host_block, uint32_t shots)
{
    g_tamper_h2d.shots.store(0);
    g_tamper_h2d.layer.store(layer);
    g_tamper_h2d.kind.store(kind);
    g_tamper_h2d.block.store(host_block);
    g_tamper_h2d.shots.store(int64_t(shots));
    return 0;
}

int secure_infer_test_tamper_d2h(uint32_t shots)
{
    g_tamper_d2h.store(int64_t(shots));
    return 0;
}

int secure_infer_d2h_batch_begin(size_t expected_tasks)
{
    if (t_batch) return -1;  // nested
    DeviceState* ds = device_state();
    if (!ds) return -1;
    t_batch = std::make_unique<D2HBatch>();
    t_batch->ds = ds;
    t_batch->expected = expected_tasks;
    return 1;
}

int secure_infer_d2h_group_begin(size_t expected_tasks)
{
    (void)expected_tasks;
    if (!t_batch || t_batch->group_open) return -1;
    t_batch->group_open = true;
    return 1;
}

int secure_infer_d2h_swap(hipStream_t stream, si_session* s, const void* dev_cache, uint64_t slot_bytes,
                          uint64_t nslots, void* host_base, uint64_t host_block_bytes, uint64_t host_nblocks,
                          const int64_t* mapping, uint32_t n, uint32_t kind, uint32_t layer,
                          uint32_t codec_bits, uint32_t heads, uint32_t head_dim)
{
    D2HBatch* b = t_batch.get();
    if (!b || !b->group_open) return -1;
    if (!s || !dev_cache || !host_base || !mapping || n == 0 || kind > 1 || nslots == 0 || host_nblocks == 0)
        return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    if (!valid_mapping(mapping, n, false, host_nblocks, nslots)) return -1;
    const si_internal::SessionKeys keys = si_internal::session_keys(s);
    if (bytes > keys.max_record_bytes) return -1;
    const uint64_t stride = secure_infer_wire_stride(bytes);

    // Joins the pending launch if it takes these records, else issues that first.
    D2HJob* J = b->pending.get();
    if (J && !(J->stream == stream && J->s == s && J->layer == layer && J->codec == codec_bits &&
               J->heads == heads && J->dim == head_dim && J->bytes == bytes && J->slot_bytes == slot_bytes &&
               J->nslots == nslots && (J->cache[kind] == nullptr || J->cache[kind] == dev_cache) &&
               !(kind == 0 && J->n > J->n_k) && (uint64_t(J->n) + n) * stride <= d2h_batch_launch_cap(*b, stride))) {
        if (d2h_issue(b) != 0) return -1;
        J = nullptr;
    }
    if (!J) {
        b->pending = std::make_unique<D2HJob>();
        J = b->pending.get();
        J->batch = b;
        J->ds = b->ds;
        J->stream = stream;
        J->s = s;
        J->hold.take(s);
        J->keys = keys;
        J->layer = layer;
        J->codec = codec_bits;
        J->heads = heads;
        J->dim = head_dim;
        J->bytes = bytes;
        J->stride = stride;
        J->tag_off = tag_offset(bytes);
        J->slot_bytes = slot_bytes;
        J->nslots = nslots;
    }
    const uint64_t t0 = si_internal::reserve_tickets(n);
    if (!si_internal::replay_reserve_range(t0, n)) {
        fprintf(stderr, "[secure_infer] duplicate D2H transfer tickets rejected at %llu\n",
                static_cast<unsigned long long>(t0));
        return -1;
    }
    // AADs (direction 2) of the host destinations, built now.
    const size_t a0 = J->aads.size();
    J->aads.resize(a0 + 64 * size_t(n));
    for (uint32_t r = 0; r < n; ++r) {
        const int64_t hb = mapping[2 * r + 1];
        uint8_t* dst = static_cast<uint8_t*>(host_base) + uint64_t(hb) * host_block_bytes;
        if (secure_infer_build_gcm_aad(dst, bytes, 2, t0 + r, 0, keys.nonce, &J->aads[a0 + 64 * size_t(r)]) != 1) {
            J->aads.resize(a0);
            return -1;
        }
    }
    for (uint32_t r = 0; r < n; ++r) {
        J->recs.push_back({static_cast<uint8_t*>(host_base) + uint64_t(mapping[2 * r + 1]) * host_block_bytes,
                           t0 + r});
        J->slot_ids.push_back(mapping[2 * r]);
    }
    J->cache[kind] = dev_cache;
    J->n += n;
    if (kind == 0) J->n_k += n;
    return 0;
}

// The group bracket is kept for the reference's callers; records of several
// groups can share a launch, issued at the latest by the batch's device
// barrier or end.
int secure_infer_d2h_group_end(void)
{
    D2HBatch* b = t_batch.get();
    if (!b || !b->group_open) return 0;
    b->group_open = false;
    return 0;
}

int secure_infer_d2h_batch_device_barrier(void)
{
    D2HBatch* b = t_batch.get();
    if (!b || b->group_open) return -1;
    if (d2h_issue(b) != 0) return -1;
    hipEvent_t join = nullptr;
    if (hipEventCreateWithFlags(&join, hipEventDisableTiming) != hipSuccess) return -1;
    b->joins.push_back(join);
    if (hipEventRecord(join, b->ds->d2h) != hipSuccess) return -1;
    for (hipStream_t st : b->streams)
        if (hipStreamWaitEvent(st, join, 0) != hipSuccess) return -1;
    return 0;
}

int secure_infer_d2h_batch_end(void)
{
    if (!t_batch) return 0;
    if (t_batch->group_open) return -1;
    std::unique_ptr<D2HBatch> b = std::move(t_batch);
    const bool issued = d2h_issue(b.get()) == 0;
    b->wait_done();
    return (issued && b->failures.load() == 0) ? 0 : -1;
}

}  // extern "C"

