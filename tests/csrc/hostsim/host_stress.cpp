// TEST INFRASTRUCTURE ONLY: a concurrency stress of the library's host
// runtime (si_host.cpp, si_api.cpp), built with the host-only HIP stand-in
// (hostsim.cpp) under ThreadSanitizer or AddressSanitizer by
// tests/test_host_sanitizers.py.  Every scenario checks its results against
// the host data (bf16 blocks, or the oracle's codec for packets) and the
// process exits non-zero at the first mismatch; the sanitizers abort at their
// first report.
//
//   reload:   threads with their own streams reload their own layers through
//             layer groups (secure_infer_h2d_swap), some sealed ahead of
//             demand (secure_infer_h2d_prefetch_group), one record corrupted
//             once (strict retry repairs it) and one corrupted twice (the
//             layer's wait fails and the slot reads as zeros); bf16 and int4;
//   store:    a thread stores every layer in one D2H batch (groups, device
//             barrier, batch_end racing the pool's verification), bf16 and
//             int8, plus a batch with a corrupted record (batch_end -1, block
//             zeroed);
//   exits:    threads that end inside a layer group and inside a D2H batch;
//   sessions: a session destroyed while its prefetches are still sealing,
//             and a destroy refused while another thread holds the session.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <memory>
#include <mutex>
#include <random>
#include <thread>
#include <vector>

#include "secure_infer_gpu.h"
#include "si_oracle.h"

extern "C" size_t hostsim_reload_log(uint32_t layer, uint64_t* out, size_t cap);

namespace {

constexpr uint32_t kHeads = 2, kDim = 64;
constexpr uint64_t kBlock = 128ull * kHeads * kDim * 2;  // bf16 block bytes
std::atomic<int> g_failures{0};

#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            fprintf(stderr, "[host_stress] FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                  \
            fprintf(stderr, "\n");                         \
            g_failures.fetch_add(1);                       \
        }                                                  \
    } while (0)

// Where each scenario thread is (a watchdog prints them if a round stalls).
constexpr int kSlots = 16;
std::atomic<const char*> g_stage[kSlots];
std::atomic<uint32_t> g_stage_layer[kSlots];

void stage(int slot, const char* what, uint32_t layer = 0)
{
    g_stage_layer[slot].store(layer);
    g_stage[slot].store(what);
}

const uint8_t kKey[16] = {0x10, 0x21, 0x32, 0x43, 0x54, 0x65, 0x76, 0x87,
                          0x98, 0xa9, 0xba, 0xcb, 0xdc, 0xed, 0xfe, 0x0f};
const uint8_t kSalt[4] = {0xca, 0xfe, 0xf0, 0x0d};

uint64_t record_bytes(uint32_t bits) { return bits ? si_or_codec_width(bits, kHeads, kDim) : kBlock; }

// n random bf16 blocks (finite, ~uniform [-4, 4)).
std::vector<uint16_t> blocks(std::mt19937& rng, size_t n)
{
    std::vector<uint16_t> v(n * kBlock / 2);
    std::uniform_real_distribution<float> d(-4.0f, 4.0f);
    for (auto& x : v) x = si_or_f32_to_bf16(d(rng));
    return v;
}

// Host pool of n records (bf16 blocks, or their packets) for (kind, layer).
std::vector<uint8_t> host_pool(const std::vector<uint16_t>& blk, size_t n, uint32_t bits, uint32_t kind,
                               uint32_t layer)
{
    const uint64_t rb = record_bytes(bits);
    std::vector<uint8_t> p(n * rb);
    for (size_t i = 0; i < n; ++i) {
        const uint16_t* b = blk.data() + i * kBlock / 2;
        if (bits) si_or_codec_encode(b, kHeads, kDim, bits, kind, layer, p.data() + i * rb);
        else memcpy(p.data() + i * rb, b, kBlock);
    }
    return p;
}

// What a reloaded slot must hold for host record `rec` (bf16 block or the
// decode of its packet).
std::vector<uint8_t> expect_slot(const uint8_t* rec, uint32_t bits, uint32_t kind)
{
    std::vector<uint8_t> out(kBlock);
    if (bits) si_or_codec_decode(rec, kHeads, kDim, bits, kind, reinterpret_cast<uint16_t*>(out.data()));
    else memcpy(out.data(), rec, kBlock);
    return out;
}

si_session* new_session(uint64_t nonce)
{
    si_session* s = nullptr;
    if (secure_infer_gpu_session_create(kKey, kSalt, nonce, record_bytes(0), &s) != 0) {
        fprintf(stderr, "[host_stress] session_create failed\n");
        exit(2);
    }
    return s;
}

// ---------------------------------------------------------------- reload

// Host buffers that must outlive the thread that handed them to the library
// (a D2H batch ended by its thread's exit still writes its destinations),
// kept until the round's threads have joined.
std::mutex g_keep_m;
std::vector<std::shared_ptr<std::vector<uint8_t>>> g_keep;

std::vector<uint8_t>& kept(std::vector<uint8_t> v)
{
    auto p = std::make_shared<std::vector<uint8_t>>(std::move(v));
    std::lock_guard<std::mutex> g(g_keep_m);
    g_keep.push_back(p);
    return *p;
}

// tamper: this thread (alone) arms the H2D fault injection for its own
// layers (it matches layer, kind and host block, so no other thread's
// records are hit).
// merge: each layer's two causal groups (tail first, as the reference's
// grouped loading submits them) go inside one layer group, K1 V1 K2 V2, so
// the launch packs K before V on the device; odd layers are sealed ahead as
// one layer buffer (secure_infer_h2d_prefetch_layer).
void reload_thread(int slot, si_session* sess, uint32_t first_layer, uint32_t layers, uint32_t bits, uint32_t seed,
                   bool tamper, bool merge)
{
    std::mt19937 rng(seed);
    hipStream_t stream;
    hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    const size_t nhost = 12, nslots = 20, n = 8;
    const uint64_t rb = record_bytes(bits);
    for (uint32_t l = 0; l < layers; ++l) {
        const uint32_t layer = first_layer + l;
        // The pools stay allocated for the round: their host ranges stay
        // registered until then, and a range found first names the record.
        std::vector<uint8_t>* pools[2];
        for (uint32_t kind = 0; kind < 2; ++kind) pools[kind] = &kept(host_pool(blocks(rng, nhost), nhost, bits, kind, layer));
        for (uint32_t kind = 0; kind < 2; ++kind)
            secure_infer_register_host_range_ex(pools[kind]->data(), pools[kind]->size(), layer, kind, rb);
        std::vector<uint8_t> cache[2];
        for (auto& c : cache) c.assign(nslots * kBlock, 0x3c);
        std::vector<int64_t> slots(nslots);
        for (size_t i = 0; i < nslots; ++i) slots[i] = int64_t(i);
        std::shuffle(slots.begin(), slots.end(), rng);
        std::vector<int64_t> map(2 * n);
        for (size_t i = 0; i < n; ++i) {
            map[2 * i] = int64_t(i + (l % 3));  // host block
            map[2 * i + 1] = slots[i];          // device slot
        }
        const int64_t victim = map[2 * 3];
        const int mode = tamper ? int(l % 4) : 0;  // 1: corrupted once, 2: corrupted twice
        if (mode == 1 || mode == 2) secure_infer_test_tamper_h2d(int32_t(layer), 1, victim, uint32_t(mode));
        stage(slot, "reload: prefetch", layer);
        // causal groups, tail first: rows [n/2, n) then [0, n/2)
        const uint32_t gstart[2] = {uint32_t(n / 2), 0}, grows[2] = {uint32_t(n - n / 2), uint32_t(n / 2)};
        if (l % 2 == 1 && merge)
            CHECK(secure_infer_h2d_prefetch_layer(sess, pools[0]->data(), pools[1]->data(), rb, nhost, map.data(), gstart,
                                                  grows, 2, layer, bits, kHeads, kDim) == 0,
                  "prefetch_layer layer %u", layer);
        else if (l % 2 == 1)
            CHECK(secure_infer_h2d_prefetch_group(sess, pools[0]->data(), pools[1]->data(), rb, nhost, map.data(),
                                                  uint32_t(n), layer, bits, kHeads, kDim) == 0,
                  "prefetch_group layer %u", layer);
        stage(slot, "reload: swaps", layer);
        CHECK(secure_infer_h2d_layer_group_begin(2 * n) == 0, "group_begin");
        if (merge) {
            for (int g = 0; g < 2; ++g)
                for (uint32_t kind = 0; kind < 2; ++kind)
                    CHECK(secure_infer_h2d_swap(stream, sess, pools[kind]->data(), rb, nhost, cache[kind].data(), kBlock,
                                                nslots, map.data() + 2 * gstart[g], grows[g], kind, layer, bits, kHeads,
                                                kDim, nullptr) == 0,
                          "h2d_swap layer %u group %d kind %u", layer, g, kind);
        } else {
            for (uint32_t kind = 0; kind < 2; ++kind)
                CHECK(secure_infer_h2d_swap(stream, sess, pools[kind]->data(), rb, nhost, cache[kind].data(), kBlock,
                                            nslots, map.data(), uint32_t(n), kind, layer, bits, kHeads, kDim,
                                            nullptr) == 0,
                      "h2d_swap layer %u kind %u", layer, kind);
        }
        stage(slot, "reload: group_end", layer);
        CHECK(secure_infer_h2d_layer_group_end() == 0, "group_end");
        stage(slot, "reload: wait_layer", layer);
        const int rc = secure_infer_recovery_wait_layer_authentication(layer);
        stage(slot, "reload: stream sync", layer);
        hipStreamSynchronize(stream);
        stage(slot, "reload: check", layer);
        {
            // Tickets rise along the reference's submission order: each causal
            // group's K records, then its V records (native_layerwise.py:96-112),
            // whether a group was its own layer group or part of a merged one,
            // sealed on demand or ahead of demand (a retry's fresh ticket is
            // later; the first ticket of each record counts).
            std::vector<uint64_t> log(3 * 4 * n * 2);
            const size_t got = hostsim_reload_log(layer, log.data(), log.size() / 3);
            std::map<std::pair<uint64_t, uint64_t>, uint64_t> first;
            for (size_t i = 0; i < std::min(got, log.size() / 3); ++i) {
                const auto key = std::make_pair(log[3 * i], log[3 * i + 1]);
                auto it = first.find(key);
                if (it == first.end() || log[3 * i + 2] < it->second) first[key] = log[3 * i + 2];
            }
            std::vector<uint64_t> seq;
            const int ngroups = merge ? 2 : 1;
            for (int g = 0; g < ngroups; ++g) {
                const uint32_t r0 = merge ? gstart[g] : 0, rows = merge ? grows[g] : uint32_t(n);
                for (uint64_t kind = 0; kind < 2; ++kind)
                    for (uint32_t r = r0; r < r0 + rows; ++r) {
                        auto it = first.find(std::make_pair(kind, uint64_t(map[2 * r])));
                        seq.push_back(it == first.end() ? 0 : it->second);
                    }
            }
            bool rising = seq.size() == 2 * n && seq[0] != 0;
            for (size_t i = 1; i < seq.size(); ++i) rising = rising && seq[i] > seq[i - 1];
            if (!rising) {
                std::string t;
                for (auto v : seq) t += " " + std::to_string(v);
                fprintf(stderr, "[host_stress] layer %u got %zu log rows, tickets:%s\n", layer, got, t.c_str());
            }
            CHECK(rising, "layer %u (merge %d, prefetched %d): tickets not in the reference's order", layer, int(merge),
                  int(l % 2 == 1));
        }
        CHECK(rc == (mode == 2 ? -1 : 0), "layer %u mode %d wait rc %d", layer, mode, rc);
        for (uint32_t kind = 0; kind < 2; ++kind)
            for (size_t i = 0; i < n; ++i) {
                const uint8_t* slot = cache[kind].data() + uint64_t(map[2 * i + 1]) * kBlock;
                if (mode == 2 && kind == 1 && map[2 * i] == victim) {
                    bool zero = true;
                    for (uint64_t b = 0; b < kBlock; ++b) zero = zero && slot[b] == 0;
                    CHECK(zero, "layer %u: the persistently corrupted record is not zeroed", layer);
                    continue;
                }
                const auto want = expect_slot(pools[kind]->data() + uint64_t(map[2 * i]) * rb, bits, kind);
                CHECK(memcmp(slot, want.data(), kBlock) == 0, "layer %u kind %u record %zu differs", layer, kind, i);
            }
        if (tamper) secure_infer_test_tamper_h2d(-1, -1, -1, 0);
    }
    stage(slot, "reload: stream destroy");
    hipStreamDestroy(stream);
    stage(slot, "reload: done");
}

// ---------------------------------------------------------------- store

void store_thread(int slot, si_session* sess, uint32_t first_layer, uint32_t layers, uint32_t bits, uint32_t seed,
                  bool tamper)
{
    std::mt19937 rng(seed);
    hipStream_t stream;
    hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    const size_t nslots = 16, nhost = 10, n = 6;
    const uint64_t rb = record_bytes(bits);
    struct Layer {
        std::vector<uint16_t> cache[2];
        std::vector<uint8_t>* pool[2];
        std::vector<int64_t> map;
    };
    std::vector<Layer> ls(layers);
    if (tamper) secure_infer_test_tamper_d2h(1);
    stage(slot, "store: swaps", first_layer);
    CHECK(secure_infer_d2h_batch_begin(2 * n * layers) == 1, "batch_begin");
    for (uint32_t l = 0; l < layers; ++l) {
        Layer& L = ls[l];
        for (uint32_t kind = 0; kind < 2; ++kind) {
            L.cache[kind] = blocks(rng, nslots);
            L.pool[kind] = &kept(std::vector<uint8_t>(nhost * rb, 0));  // registered until the round ends
            secure_infer_register_host_range_ex(L.pool[kind]->data(), L.pool[kind]->size(), first_layer + l, kind, rb);
        }
        L.map.resize(2 * n);
        for (size_t i = 0; i < n; ++i) {
            L.map[2 * i] = int64_t((i * 5 + l) % nslots);  // device slot
            L.map[2 * i + 1] = int64_t(i + 2);             // host block
        }
        for (uint32_t kind = 0; kind < 2; ++kind) {
            CHECK(secure_infer_d2h_group_begin(n) == 1, "d2h group_begin");
            CHECK(secure_infer_d2h_swap(stream, sess, L.cache[kind].data(), kBlock, nslots, L.pool[kind]->data(), rb,
                                        nhost, L.map.data(), uint32_t(n), kind, first_layer + l, bits, kHeads,
                                        kDim) == 0,
                  "d2h_swap");
            CHECK(secure_infer_d2h_group_end() == 0, "d2h group_end");
        }
    }
    stage(slot, "store: device barrier", first_layer);
    CHECK(secure_infer_d2h_batch_device_barrier() == 0, "device barrier");
    stage(slot, "store: batch_end", first_layer);
    const int rc = secure_infer_d2h_batch_end();
    stage(slot, "store: check", first_layer);
    CHECK(rc == (tamper ? -1 : 0), "batch_end rc %d (tamper %d)", rc, int(tamper));
    size_t zeroed = 0;
    for (uint32_t l = 0; l < layers; ++l) {
        Layer& L = ls[l];
        for (uint32_t kind = 0; kind < 2; ++kind)
            for (size_t i = 0; i < n; ++i) {
                const uint8_t* got = L.pool[kind]->data() + uint64_t(L.map[2 * i + 1]) * rb;
                std::vector<uint8_t> want(rb);
                const uint16_t* blk = L.cache[kind].data() + uint64_t(L.map[2 * i]) * kBlock / 2;
                if (bits) si_or_codec_encode(blk, kHeads, kDim, bits, kind, first_layer + l, want.data());
                else memcpy(want.data(), blk, kBlock);
                if (memcmp(got, want.data(), rb) == 0) continue;
                bool zero = true;
                for (uint64_t b = 0; b < rb; ++b) zero = zero && got[b] == 0;
                CHECK(tamper && zero, "layer %u kind %u block %zu differs", first_layer + l, kind, i);
                ++zeroed;
            }
    }
    CHECK(zeroed == (tamper ? 1u : 0u), "%zu zeroed blocks (tamper %d)", zeroed, int(tamper));
    secure_infer_test_tamper_d2h(0);
    stage(slot, "store: stream destroy", first_layer);
    hipStreamDestroy(stream);
    stage(slot, "store: done");
}

// ---------------------------------------------------------------- exits

// A thread ends inside a layer group with a swap queued: its ring slot and
// session hold go with it; nothing was issued.
void exit_inside_group(int slot, si_session* sess, uint32_t layer, uint32_t seed)
{
    stage(slot, "exit_inside_group: start", layer);
    std::mt19937 rng(seed);
    hipStream_t stream;
    hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    auto& pool = kept(host_pool(blocks(rng, 4), 4, 0, 0, layer));
    secure_infer_register_host_range_ex(pool.data(), pool.size(), layer, 0, kBlock);
    auto& cache = kept(std::vector<uint8_t>(4 * kBlock, 0));
    const int64_t map[4] = {0, 1, 2, 3};
    CHECK(secure_infer_h2d_layer_group_begin(4) == 0, "group_begin");
    CHECK(secure_infer_h2d_swap(stream, sess, pool.data(), kBlock, 4, cache.data(), kBlock, 4, map, 2, 0, layer, 0,
                                kHeads, kDim, nullptr) == 0,
          "swap");
    // no group_end: the thread ends here (its stream outlives it)
    stage(slot, "exit_inside_group: thread exit", layer);
}

// A thread ends inside a D2H batch: its issued launches finish first.
void exit_inside_batch(int slot, si_session* sess, uint32_t layer, uint32_t seed)
{
    stage(slot, "exit_inside_batch: start", layer);
    std::mt19937 rng(seed);
    static hipStream_t stream = [] {
        hipStream_t s;
        hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        return s;
    }();
    const auto blk = blocks(rng, 4);
    auto& cache = kept(std::vector<uint8_t>(reinterpret_cast<const uint8_t*>(blk.data()),
                                            reinterpret_cast<const uint8_t*>(blk.data()) + 4 * kBlock));
    auto& pool = kept(std::vector<uint8_t>(4 * kBlock, 0));
    secure_infer_register_host_range_ex(pool.data(), pool.size(), layer, 0, kBlock);
    const int64_t map[4] = {0, 1, 2, 3};
    CHECK(secure_infer_d2h_batch_begin(2) == 1, "batch_begin");
    CHECK(secure_infer_d2h_group_begin(2) == 1, "group_begin");
    CHECK(secure_infer_d2h_swap(stream, sess, cache.data(), kBlock, 4, pool.data(), kBlock, 4, map, 2, 0, layer, 0,
                                kHeads, kDim) == 0,
          "swap");
    CHECK(secure_infer_d2h_group_end() == 0, "group_end");
    CHECK(secure_infer_d2h_batch_device_barrier() == 0, "barrier");  // issues the launch
    // no batch_end: the thread's batch waits for its launch as the thread ends
    stage(slot, "exit_inside_batch: thread exit", layer);
}

// ---------------------------------------------------------------- sessions

void destroy_during_prefetch(int slot, uint32_t layer, uint32_t seed)
{
    stage(slot, "destroy_during_prefetch: prefetch", layer);
    std::mt19937 rng(seed);
    si_session* s = new_session(900 + seed);
    const size_t nhost = 16, n = 16;
    auto& k = kept(host_pool(blocks(rng, nhost), nhost, 0, 0, layer));
    auto& v = kept(host_pool(blocks(rng, nhost), nhost, 0, 1, layer));
    secure_infer_register_host_range_ex(k.data(), k.size(), layer, 0, kBlock);
    secure_infer_register_host_range_ex(v.data(), v.size(), layer, 1, kBlock);
    std::vector<int64_t> map(2 * n);
    for (size_t i = 0; i < n; ++i) {
        map[2 * i] = int64_t(i);
        map[2 * i + 1] = int64_t(i);
    }
    for (int rep = 0; rep < 4; ++rep)
        CHECK(secure_infer_h2d_prefetch_group(s, k.data(), v.data(), kBlock, nhost, map.data(), uint32_t(n), layer, 0,
                                              kHeads, kDim) == 0,
              "prefetch");
    stage(slot, "destroy_during_prefetch: destroy", layer);
    CHECK(secure_infer_gpu_session_destroy(s) == 0, "destroy with prefetches sealing");
    stage(slot, "destroy_during_prefetch: done", layer);
}

void destroy_refused_while_held(uint32_t layer, uint32_t seed)
{
    std::mt19937 rng(seed);
    si_session* s = new_session(1700 + seed);
    auto& pool = kept(host_pool(blocks(rng, 4), 4, 0, 0, layer));
    secure_infer_register_host_range_ex(pool.data(), pool.size(), layer, 0, kBlock);
    std::vector<uint8_t> cache(4 * kBlock, 0);
    std::atomic<int> step{0};
    hipStream_t stream;
    hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    std::thread holder([&] {
        const int64_t map[4] = {0, 1, 2, 3};
        CHECK(secure_infer_h2d_layer_group_begin(2) == 0, "group_begin");
        CHECK(secure_infer_h2d_swap(stream, s, pool.data(), kBlock, 4, cache.data(), kBlock, 4, map, 2, 0, layer, 0,
                                    kHeads, kDim, nullptr) == 0,
              "swap");
        step.store(1);
        while (step.load() != 2) std::this_thread::yield();
        CHECK(secure_infer_h2d_layer_group_end() == 0, "group_end");
        CHECK(secure_infer_recovery_wait_layer_authentication(layer) == 0, "wait");
    });
    while (step.load() != 1) std::this_thread::yield();
    CHECK(secure_infer_gpu_session_destroy(s) == -1, "destroy must be refused while another thread holds it");
    step.store(2);
    holder.join();
    hipStreamSynchronize(stream);
    CHECK(memcmp(cache.data() + kBlock, pool.data(), kBlock) == 0 &&
              memcmp(cache.data() + 3 * kBlock, pool.data() + 2 * kBlock, kBlock) == 0,
          "held session's reload differs");
    CHECK(secure_infer_gpu_session_destroy(s) == 0, "destroy after release");
    hipStreamDestroy(stream);
}

}  // namespace

// Prints every thread's stage and aborts when a round makes no progress for
// `limit` seconds (a hang in the library or the stand-in shows where).
std::atomic<int> g_round_done{-1};

void watchdog(int rounds, int limit)
{
    int last = -1;
    auto since = std::chrono::steady_clock::now();
    while (g_round_done.load() < rounds - 1) {
        std::this_thread::sleep_for(std::chrono::milliseconds(200));
        const int now = g_round_done.load();
        if (now != last) {
            last = now;
            since = std::chrono::steady_clock::now();
        } else if (std::chrono::steady_clock::now() - since > std::chrono::seconds(limit)) {
            fprintf(stderr, "[host_stress] WATCHDOG: round %d stalled for %d s\n", now + 1, limit);
            for (int i = 0; i < kSlots; ++i) {
                const char* st = g_stage[i].load();
                if (st) fprintf(stderr, "  thread slot %d: %s (layer %u)\n", i, st, g_stage_layer[i].load());
            }
            fflush(stderr);
            abort();
        }
    }
}

int main(int argc, char** argv)
{
    if (argc > 1 && std::string(argv[1]) == "d2h_failure") {
        // One store batch with one record corrupted on its way to the host:
        // the batch fails (batch_end -1, the block zeroed), or, with
        // SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE=1, the process aborts first.
        si_session* sess = new_session(4242);
        store_thread(0, sess, 5000, 1, 0u, 99u, true);
        CHECK(secure_infer_gpu_session_destroy(sess) == 0, "destroy");
        hipDeviceSynchronize();
        if (g_failures.load()) return 1;
        printf("D2H_FAILURE_REPORTED\n");
        return 0;
    }
    const int rounds = argc > 1 ? atoi(argv[1]) : 2;
    const int limit = argc > 2 ? atoi(argv[2]) : 60;
    std::thread dog(watchdog, rounds, limit);
    si_session* sess = new_session(77);
    for (int round = 0; round < rounds; ++round) {
        const uint32_t base = 1000u * uint32_t(round + 1);
        for (int i = 0; i < kSlots; ++i) g_stage[i].store(nullptr);
        std::vector<std::thread> ts;
        ts.emplace_back(reload_thread, 0, sess, base + 0, 8, 0u, 11u + round, true, false);
        ts.emplace_back(reload_thread, 1, sess, base + 100, 8, 4u, 12u + round, false, false);
        ts.emplace_back(reload_thread, 2, sess, base + 200, 6, 0u, 13u + round, false, false);
        ts.emplace_back(store_thread, 3, sess, base + 300, 5, 0u, 14u + round, false);
        ts.emplace_back(store_thread, 4, sess, base + 400, 4, 8u, 15u + round, false);
        ts.emplace_back(reload_thread, 11, sess, base + 650, 8, 4u, 22u + round, false, true);
        ts.emplace_back(exit_inside_group, 5, sess, base + 600, 17u + round);
        ts.emplace_back(exit_inside_batch, 6, sess, base + 700, 18u + round);
        ts.emplace_back(destroy_during_prefetch, 7, base + 800, 19u + round);
        for (auto& t : ts) t.join();
        // The D2H fault injection hits any record: the tampered store runs
        // with no other store in flight, beside more reloads.
        stage(10, "main: tampered store phase");
        std::thread tr(reload_thread, 8, sess, base + 250, 8, 0u, 21u + round, true, true);
        store_thread(9, sess, base + 500, 3, 0u, 16u + round, true);
        tr.join();
        stage(10, "main: destroy_refused_while_held");
        destroy_refused_while_held(base + 900, 20u + round);
        stage(10, "main: round end");
        secure_infer_clear_host_ranges();
        {
            std::lock_guard<std::mutex> g(g_keep_m);
            g_keep.clear();
        }
        fprintf(stderr, "[host_stress] round %d done, %d failures\n", round, g_failures.load());
        g_round_done.store(round);
    }
    dog.join();
    CHECK(secure_infer_gpu_session_destroy(sess) == 0, "final destroy");
    hipDeviceSynchronize();
    if (g_failures.load()) {
        fprintf(stderr, "[host_stress] %d FAILURES\n", g_failures.load());
        return 1;
    }
    printf("HOST_STRESS_OK rounds=%d\n", rounds);
    return 0;
}
