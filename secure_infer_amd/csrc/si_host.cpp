// Host side of the authenticated transfer path on MI355X.
//
//  * A worker pool runs OpenSSL AES-128-GCM (EVP, one context per thread) --
//    the reference's host crypto (inline_h2d_encrypt_commit,
//    secure_infer.cpp:6486-6550; d2h_host_decrypt_one, :2470-2547).
//  * H2D: secure_infer_h2d_swap seals host KV blocks into wire records in a
//    pinned ring slot, copies the slot to the device on the library's copy
//    stream and makes the caller's stream wait for that copy before the fused
//    verify + decrypt (+ dequant) + paged-scatter kernel.  The caller returns
//    as soon as the work is queued, so the copy of layer l+1 overlaps the
//    kernel of layer l.  A slot is reused only after its kernel completed.
//  * D2H: the reference's batch / group API with the same names and
//    thread-local contexts (secure_infer.cpp:2707-2970).  Inside a group,
//    secure_infer_d2h_swap gathers (+ quantises) and seals device KV blocks
//    on the caller's stream, then copies the records to pinned memory on a
//    second copy stream; the group's end hands them to the worker pool, which
//    authenticates and decrypts each record into its host destination (a
//    record that fails is zeroed).  batch_end waits for that verification.
#include "si_host.h"

#include <openssl/evp.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
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
        }
        cv_.notify_one();
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
        const size_t helpers = std::min(threads_.size(), n - 1);
        for (size_t h = 0; h < helpers; ++h) submit(body);
        body();
        std::unique_lock<std::mutex> g(sh->m);
        sh->cv.wait(g, [&] { return sh->done.load() == n; });
    }

private:
    Pool()
    {
        // CPUs this process may run on (the affinity mask, not the machine).
        unsigned n = std::thread::hardware_concurrency();
        cpu_set_t set;
        CPU_ZERO(&set);
        if (sched_getaffinity(0, sizeof(set), &set) == 0) n = unsigned(CPU_COUNT(&set));
        if (const char* e = std::getenv("SECURE_INFER_HOST_THREADS")) n = unsigned(std::atoi(e));
        if (n == 0) n = 1;
        if (n > 64) n = 64;
        for (unsigned i = 0; i + 1 < n; ++i) threads_.emplace_back([this] { run(); });
    }

    void run()
    {
        for (;;) {
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> g(m_);
                cv_.wait(g, [&] { return !q_.empty(); });
                f = std::move(q_.front());
                q_.pop_front();
            }
            f();
        }
    }

public:
    size_t threads() const { return threads_.size() + 1; }

private:
    std::vector<std::thread> threads_;
    std::deque<std::function<void()>> q_;
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

// ---------------------------------------------------------------- device buffers

// A pinned host buffer mirrored by a device buffer of the same size, plus
// device scratch for codec packets, reused across calls.
struct Mirror {
    uint8_t* host = nullptr;
    uint8_t* dev = nullptr;
    size_t cap = 0;
    uint8_t* stage = nullptr;
    size_t stage_cap = 0;
    hipEvent_t ev_a = nullptr, ev_b = nullptr;

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

struct DeviceState {
    hipStream_t h2d = nullptr;  // H2D copies of the reload ring
    hipStream_t d2h = nullptr;  // D2H copies of sealed records
    std::mutex ring_lock;
    std::vector<std::unique_ptr<Mirror>> ring;
    std::vector<bool> ring_used;
    size_t next = 0;
    std::mutex pool_lock;
    std::vector<std::unique_ptr<Mirror>> free_bufs;  // D2H buffers between batches
};

DeviceState* device_state()
{
    static std::mutex m;
    static std::map<int, std::unique_ptr<DeviceState>> states;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> g(m);
    auto& st = states[dev];
    if (!st) {
        auto s = std::make_unique<DeviceState>();
        // default priority on purpose: every stream of the library shares it
        if (hipStreamCreateWithFlags(&s->h2d, hipStreamNonBlocking) != hipSuccess ||
            hipStreamCreateWithFlags(&s->d2h, hipStreamNonBlocking) != hipSuccess)
            return nullptr;
        size_t slots = 4;
        if (const char* e = std::getenv("SECURE_INFER_H2D_SLOTS")) slots = size_t(std::max(2, std::atoi(e)));
        for (size_t i = 0; i < slots; ++i) {
            auto mbuf = std::make_unique<Mirror>();
            if (!mbuf->init()) return nullptr;
            s->ring.push_back(std::move(mbuf));
            s->ring_used.push_back(false);
        }
        st = std::move(s);
    }
    return st.get();
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

// ---------------------------------------------------------------- D2H batches

struct D2HJob {
    std::unique_ptr<Mirror> buf;
    uint32_t n = 0;
    uint64_t bytes = 0, stride = 0, tag_off = 0, t0 = 0;
    uint8_t* host_base = nullptr;
    uint64_t host_block_bytes = 0;
    std::vector<int64_t> host_blocks;
    si_internal::SessionKeys keys{};
};

struct D2HBatch {
    DeviceState* ds = nullptr;
    bool group_open = false;
    std::vector<std::unique_ptr<D2HJob>> jobs;
    size_t group_first = 0;  // first job of the open group
    std::vector<hipStream_t> streams;
    std::vector<hipEvent_t> joins;
    std::atomic<size_t> pending{0};
    std::atomic<uint64_t> failures{0};
    std::mutex m;
    std::condition_variable cv;
};

thread_local std::unique_ptr<D2HBatch> t_batch;

std::unique_ptr<Mirror> take_buffer(DeviceState* ds)
{
    {
        std::lock_guard<std::mutex> g(ds->pool_lock);
        if (!ds->free_bufs.empty()) {
            auto b = std::move(ds->free_bufs.back());
            ds->free_bufs.pop_back();
            return b;
        }
    }
    auto b = std::make_unique<Mirror>();
    if (!b->init()) return nullptr;
    return b;
}

void verify_records(D2HBatch* b, D2HJob* job, uint32_t r0, uint32_t r1)
{
    uint64_t bad = 0;
    if (hipEventSynchronize(job->buf->ev_b) != hipSuccess) {
        bad = r1 - r0;
    } else {
        for (uint32_t r = r0; r < r1; ++r) {
            const uint8_t* rec = job->buf->host + uint64_t(r) * job->stride;
            uint8_t* dst = job->host_base + uint64_t(job->host_blocks[r]) * job->host_block_bytes;
            uint8_t iv[12];
            record_iv(job->keys, job->t0 + r, iv);
            if (!gcm_open(job->keys.key, iv, rec + job->tag_off + 32, 64, rec, job->bytes,
                          rec + job->tag_off, dst)) {
                memset(dst, 0, job->bytes);  // fail closed
                ++bad;
            }
        }
    }
    if (bad) b->failures.fetch_add(bad);
    if (b->pending.fetch_sub(1) == 1) {
        std::lock_guard<std::mutex> g(b->m);
        b->cv.notify_all();
    }
}

}  // namespace

extern "C" {

int secure_infer_host_threads(void) { return int(Pool::get().threads()); }

int secure_infer_h2d_swap(hipStream_t stream, si_session* s, const void* host_base,
                          uint64_t host_block_bytes, void* dev_cache, uint64_t slot_bytes,
                          uint64_t nslots, const int64_t* mapping, uint32_t n, uint32_t kind,
                          uint32_t layer, uint32_t codec_bits, uint32_t heads, uint32_t head_dim,
                          uint32_t* fail_count)
{
    if (!s || !host_base || !dev_cache || !mapping || n == 0 || kind > 1 || nslots == 0) return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    const si_internal::SessionKeys keys = si_internal::session_keys(s);
    if (bytes > keys.max_record_bytes) return -1;
    DeviceState* ds = device_state();
    if (!ds) return -1;
    const uint64_t stride = secure_infer_wire_stride(bytes);
    const uint64_t tag_off = tag_offset(bytes);
    const size_t wire = size_t(n) * stride;
    const size_t need = wire + size_t(n) * 8;

    std::lock_guard<std::mutex> g(ds->ring_lock);
    const size_t si = ds->next;
    ds->next = (ds->next + 1) % ds->ring.size();
    Mirror& sl = *ds->ring[si];
    if (ds->ring_used[si] && hipEventSynchronize(sl.ev_b) != hipSuccess) return -1;
    if (!sl.reserve(need, codec_bits ? size_t(n) * tag_off : 0)) return -1;

    const uint64_t t0 = si_internal::reserve_tickets(n);
    int64_t* slot_ids = reinterpret_cast<int64_t*>(sl.host + wire);
    std::atomic<int> bad{0};
    Pool::get().parallel_for(n, [&](size_t r) {
        const int64_t hb = mapping[2 * r];
        slot_ids[r] = mapping[2 * r + 1];
        uint8_t* rec = sl.host + r * stride;
        if (hb < 0) {
            bad.store(1);
            return;
        }
        const uint8_t* src = static_cast<const uint8_t*>(host_base) + uint64_t(hb) * host_block_bytes;
        uint8_t* aad = rec + tag_off + 32;
        uint8_t iv[12];
        record_iv(keys, t0 + r, iv);
        if (secure_infer_build_gcm_aad(src, bytes, 1, t0 + r, 0, keys.nonce, aad) != 1 ||
            !gcm_seal(keys.key, iv, aad, 64, src, bytes, rec, rec + tag_off)) {
            bad.store(1);
            return;
        }
        memset(rec + bytes, 0, tag_off - bytes);
        memset(rec + tag_off + 16, 0, 16);  // status slot
    });
    if (bad.load()) return -1;
    if (hipMemcpyAsync(sl.dev, sl.host, need, hipMemcpyHostToDevice, ds->h2d) != hipSuccess ||
        hipEventRecord(sl.ev_a, ds->h2d) != hipSuccess || hipStreamWaitEvent(stream, sl.ev_a, 0) != hipSuccess)
        return -1;
    si_reload_desc d{};
    d.wire = sl.dev;
    d.wire_stride = stride;
    d.bytes = bytes;
    d.nrec = n;
    d.n_k = kind == 0 ? n : 0;
    d.iv_words = nullptr;
    d.ticket_base = t0;
    d.cache_k = dev_cache;
    d.cache_v = dev_cache;
    d.slot_bytes = slot_bytes;
    d.nslots = nslots;
    d.slots = reinterpret_cast<const int64_t*>(sl.dev + wire);
    d.codec_bits = codec_bits;
    d.heads = heads;
    d.head_dim = head_dim;
    d.layer = layer;
    d.staging = sl.stage;
    d.fail_count = fail_count;
    if (secure_infer_gpu_reload_layer(stream, s, &d) != 0) return -1;
    if (hipEventRecord(sl.ev_b, stream) != hipSuccess) return -1;
    ds->ring_used[si] = true;
    si_internal::group_note(stream, layer, fail_count);
    return 0;
}

int secure_infer_d2h_batch_begin(size_t expected_tasks)
{
    (void)expected_tasks;
    if (t_batch) return -1;  // nested
    DeviceState* ds = device_state();
    if (!ds) return -1;
    t_batch = std::make_unique<D2HBatch>();
    t_batch->ds = ds;
    return 1;
}

int secure_infer_d2h_group_begin(size_t expected_tasks)
{
    (void)expected_tasks;
    if (!t_batch || t_batch->group_open) return -1;
    t_batch->group_open = true;
    t_batch->group_first = t_batch->jobs.size();
    return 1;
}

int secure_infer_d2h_swap(hipStream_t stream, si_session* s, const void* dev_cache, uint64_t slot_bytes,
                          uint64_t nslots, void* host_base, uint64_t host_block_bytes,
                          const int64_t* mapping, uint32_t n, uint32_t kind, uint32_t layer,
                          uint32_t codec_bits, uint32_t heads, uint32_t head_dim)
{
    D2HBatch* b = t_batch.get();
    if (!b || !b->group_open) return -1;
    if (!s || !dev_cache || !host_base || !mapping || n == 0 || kind > 1 || nslots == 0) return -1;
    uint64_t bytes = 0;
    if (!valid_geometry(codec_bits, heads, head_dim, host_block_bytes, bytes)) return -1;
    auto job = std::make_unique<D2HJob>();
    job->keys = si_internal::session_keys(s);
    if (bytes > job->keys.max_record_bytes) return -1;
    job->buf = take_buffer(b->ds);
    if (!job->buf) return -1;
    job->n = n;
    job->bytes = bytes;
    job->stride = secure_infer_wire_stride(bytes);
    job->tag_off = tag_offset(bytes);
    job->host_base = static_cast<uint8_t*>(host_base);
    job->host_block_bytes = host_block_bytes;
    job->host_blocks.resize(n);
    const size_t wire = size_t(n) * job->stride;
    if (!job->buf->reserve(wire + size_t(n) * 8, codec_bits ? size_t(n) * job->tag_off : 0)) return -1;
    job->t0 = si_internal::reserve_tickets(n);

    // AADs (direction 2) and device slot ids go up first, on the caller's stream.
    uint8_t* h = job->buf->host;
    int64_t* slot_ids = reinterpret_cast<int64_t*>(h + wire);
    for (uint32_t r = 0; r < n; ++r) {
        const int64_t ds_id = mapping[2 * r], hb = mapping[2 * r + 1];
        if (hb < 0) return -1;
        slot_ids[r] = ds_id;
        job->host_blocks[r] = hb;
        const uint8_t* dst = job->host_base + uint64_t(hb) * host_block_bytes;
        if (secure_infer_build_gcm_aad(dst, bytes, 2, job->t0 + r, 0, job->keys.nonce,
                                       h + uint64_t(r) * job->stride + job->tag_off + 32) != 1)
            return -1;
    }
    uint8_t* d = job->buf->dev;
    if (hipMemcpy2DAsync(d + job->tag_off + 32, job->stride, h + job->tag_off + 32, job->stride, 64, n,
                         hipMemcpyHostToDevice, stream) != hipSuccess ||
        hipMemcpyAsync(d + wire, h + wire, size_t(n) * 8, hipMemcpyHostToDevice, stream) != hipSuccess)
        return -1;
    si_writeback_desc w{};
    w.wire = d;
    w.wire_stride = job->stride;
    w.bytes = bytes;
    w.nrec = n;
    w.n_k = kind == 0 ? n : 0;
    w.iv_words = nullptr;
    w.ticket_base = job->t0;
    w.cache_k = dev_cache;
    w.cache_v = dev_cache;
    w.slot_bytes = slot_bytes;
    w.nslots = nslots;
    w.slots = reinterpret_cast<const int64_t*>(d + wire);
    w.codec_bits = codec_bits;
    w.heads = heads;
    w.head_dim = head_dim;
    w.layer = layer;
    w.staging = job->buf->stage;
    w.fail_count = nullptr;
    if (secure_infer_gpu_writeback_layer(stream, s, &w) != 0) return -1;
    DeviceState* ds = b->ds;
    if (hipEventRecord(job->buf->ev_a, stream) != hipSuccess ||
        hipStreamWaitEvent(ds->d2h, job->buf->ev_a, 0) != hipSuccess ||
        hipMemcpyAsync(h, d, wire, hipMemcpyDeviceToHost, ds->d2h) != hipSuccess ||
        hipEventRecord(job->buf->ev_b, ds->d2h) != hipSuccess)
        return -1;
    if (std::find(b->streams.begin(), b->streams.end(), stream) == b->streams.end())
        b->streams.push_back(stream);
    b->jobs.push_back(std::move(job));
    return 0;
}

int secure_infer_d2h_group_end(void)
{
    D2HBatch* b = t_batch.get();
    if (!b || !b->group_open) return 0;
    b->group_open = false;
    const uint32_t per_task = 4;
    for (size_t j = b->group_first; j < b->jobs.size(); ++j) {
        D2HJob* job = b->jobs[j].get();
        for (uint32_t r0 = 0; r0 < job->n; r0 += per_task) {
            const uint32_t r1 = std::min(job->n, r0 + per_task);
            b->pending.fetch_add(1);
            Pool::get().submit([b, job, r0, r1] { verify_records(b, job, r0, r1); });
        }
    }
    return 0;
}

int secure_infer_d2h_batch_device_barrier(void)
{
    D2HBatch* b = t_batch.get();
    if (!b || b->group_open) return -1;
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
    {
        std::unique_lock<std::mutex> g(b->m);
        b->cv.wait(g, [&] { return b->pending.load() == 0; });
    }
    for (hipEvent_t e : b->joins) {
        (void)hipEventSynchronize(e);
        (void)hipEventDestroy(e);
    }
    {
        std::lock_guard<std::mutex> g(b->ds->pool_lock);
        for (auto& job : b->jobs) b->ds->free_bufs.push_back(std::move(job->buf));
    }
    return b->failures.load() ? -1 : 0;
}

}  // extern "C"
