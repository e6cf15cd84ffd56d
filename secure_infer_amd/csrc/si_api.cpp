// libsecure_infer.so host side: per-key GCM contexts, sessions, ticket / IV /
// AAD bookkeeping and the C-ABI declared in include/secure_infer_gpu.h.
#include "secure_infer_gpu.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <initializer_list>
#include <utility>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "si_layout.h"
#include "si_host.h"
#include "si_kernels.h"

#include <openssl/core_names.h>
#include <openssl/crypto.h>
#include <openssl/evp.h>
#include <openssl/params.h>
#include <openssl/rand.h>

namespace {

// ---------------------------------------------------------------- AES (host)
// FIPS-197; the S-box is derived from GF(2^8) inversion and the affine map.

uint8_t gf8_mul(uint8_t a, uint8_t b)
{
    uint8_t r = 0;
    while (b) {
        if (b & 1) r ^= a;
        a = uint8_t((a << 1) ^ ((a & 0x80) ? 0x1b : 0));
        b >>= 1;
    }
    return r;
}

struct Sbox {
    uint8_t s[256];
    Sbox()
    {
        for (int x = 0; x < 256; ++x) {
            uint8_t inv = 0;
            if (x) {
                uint8_t p = uint8_t(x), acc = 1;
                for (int e = 254; e; e >>= 1) {
                    if (e & 1) acc = gf8_mul(acc, p);
                    p = gf8_mul(p, p);
                }
                inv = acc;
            }
            uint8_t b = inv, r = inv;
            for (int k = 1; k <= 4; ++k) {
                b = uint8_t((b << 1) | (b >> 7));
                r ^= b;
            }
            s[x] = uint8_t(r ^ 0x63);
        }
    }
};
const Sbox& sbox()
{
    static const Sbox s;
    return s;
}

void aes_expand(const uint8_t key[16], uint8_t rk[176])
{
    const uint8_t* S = sbox().s;
    memcpy(rk, key, 16);
    uint8_t rcon = 1;
    for (int i = 4; i < 44; ++i) {
        uint8_t t[4];
        memcpy(t, rk + 4 * (i - 1), 4);
        if ((i & 3) == 0) {
            const uint8_t f = t[0];
            t[0] = uint8_t(S[t[1]] ^ rcon);
            t[1] = S[t[2]];
            t[2] = S[t[3]];
            t[3] = S[f];
            rcon = gf8_mul(rcon, 2);
        }
        for (int j = 0; j < 4; ++j) rk[4 * i + j] = uint8_t(rk[4 * (i - 4) + j] ^ t[j]);
    }
}

void aes_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16])
{
    const uint8_t* S = sbox().s;
    uint8_t s[16], t[16];
    for (int i = 0; i < 16; ++i) s[i] = uint8_t(in[i] ^ rk[i]);
    for (int round = 1; round <= 10; ++round) {
        for (int c = 0; c < 4; ++c)
            for (int r = 0; r < 4; ++r) t[r + 4 * c] = S[s[r + 4 * ((c + r) & 3)]];
        if (round < 10) {
            for (int c = 0; c < 4; ++c) {
                const uint8_t* a = t + 4 * c;
                s[4 * c + 0] = uint8_t(gf8_mul(a[0], 2) ^ gf8_mul(a[1], 3) ^ a[2] ^ a[3]);
                s[4 * c + 1] = uint8_t(a[0] ^ gf8_mul(a[1], 2) ^ gf8_mul(a[2], 3) ^ a[3]);
                s[4 * c + 2] = uint8_t(a[0] ^ a[1] ^ gf8_mul(a[2], 2) ^ gf8_mul(a[3], 3));
                s[4 * c + 3] = uint8_t(gf8_mul(a[0], 3) ^ a[1] ^ a[2] ^ gf8_mul(a[3], 2));
            }
        } else {
            memcpy(s, t, 16);
        }
        for (int i = 0; i < 16; ++i) s[i] ^= rk[16 * round + i];
    }
    memcpy(out, s, 16);
}

uint32_t le32(const uint8_t* p) { return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; }
uint32_t be32(const uint8_t* p) { return uint32_t(p[0]) << 24 | uint32_t(p[1]) << 16 | uint32_t(p[2]) << 8 | uint32_t(p[3]); }
void put_be32(uint8_t* p, uint32_t v) { p[0] = uint8_t(v >> 24); p[1] = uint8_t(v >> 16); p[2] = uint8_t(v >> 8); p[3] = uint8_t(v); }
void put_be64(uint8_t* p, uint64_t v) { for (int i = 0; i < 8; ++i) p[i] = uint8_t(v >> (56 - 8 * i)); }

// ---------------------------------------------------------------- GF(2^128) (host)
// Elements as 16 bytes in GCM order (bit 0 = MSB of byte 0 = x^0).

struct Blk {
    uint8_t b[16];
};

Blk gf_mul(const Blk& x, const Blk& y)
{
    // right-shift multiply (SP 800-38D Algorithm 1) on two 64-bit halves
    uint64_t vh = 0, vl = 0, zh = 0, zl = 0;
    for (int i = 0; i < 8; ++i) {
        vh = vh << 8 | y.b[i];
        vl = vl << 8 | y.b[8 + i];
    }
    for (int i = 0; i < 128; ++i) {
        if ((x.b[i >> 3] >> (7 - (i & 7))) & 1) {
            zh ^= vh;
            zl ^= vl;
        }
        const uint64_t lsb = vl & 1;
        vl = (vl >> 1) | (vh << 63);
        vh >>= 1;
        if (lsb) vh ^= 0xe100000000000000ull;
    }
    Blk z;
    for (int i = 0; i < 8; ++i) {
        z.b[i] = uint8_t(zh >> (56 - 8 * i));
        z.b[8 + i] = uint8_t(zl >> (56 - 8 * i));
    }
    return z;
}

// Fast multiply by one fixed element with 16 per-nibble-position tables.
struct FixedMul {
    Blk t[32][16];
    explicit FixedMul(const Blk& h)
    {
        for (int p = 0; p < 32; ++p)
            for (int v = 0; v < 16; ++v) {
                Blk x{};
                x.b[p >> 1] = uint8_t((p & 1) ? v << 4 : v);
                t[p][v] = gf_mul(x, h);
            }
    }
    Blk operator()(const Blk& x) const
    {
        Blk z{};
        for (int p = 0; p < 32; ++p) {
            const int v = (x.b[p >> 1] >> ((p & 1) * 4)) & 15;
            for (int k = 0; k < 16; ++k) z.b[k] ^= t[p][v].b[k];
        }
        return z;
    }
};

// ---------------------------------------------------------------- contexts

// A session's device context and the host's copies of its key and H.  Both
// are wiped when the context goes (the device copy holds the round keys).
struct DevCtx {
    si::GcmCtx* dev = nullptr;
    uint32_t npow = 0;
    uint8_t key[16];
    uint8_t h[16];
    // L * H of the last few record shapes (L = the length block): it reveals
    // H, so it lives and dies with the context rather than in a launch cache.
    struct Lh {
        uint64_t bytes, aad_bytes;
        uint32_t w[4];
    };
    std::mutex lh_m;
    Lh lh[4]{};
    int lh_used = 0, lh_next = 0;
    void lh_of(uint64_t bytes, uint64_t aad_bytes, uint32_t out[4]);
    ~DevCtx()
    {
        if (dev) {
            (void)hipMemset(dev, 0, sizeof(si::GcmCtx) + size_t(npow) * 16);
            (void)hipFree(dev);
        }
        OPENSSL_cleanse(key, sizeof(key));
        OPENSSL_cleanse(h, sizeof(h));
        OPENSSL_cleanse(lh, sizeof(lh));
    }
};

void DevCtx::lh_of(uint64_t bytes, uint64_t aad_bytes, uint32_t out[4])
{
    std::lock_guard<std::mutex> g(lh_m);
    for (int i = 0; i < lh_used; ++i)
        if (lh[i].bytes == bytes && lh[i].aad_bytes == aad_bytes) {
            memcpy(out, lh[i].w, 16);
            return;
        }
    Blk len{}, hb;
    put_be64(len.b, aad_bytes * 8u);
    put_be64(len.b + 8, bytes * 8u);
    memcpy(hb.b, h, 16);
    Blk r = gf_mul(len, hb);
    Lh& e = lh[lh_next];
    e.bytes = bytes;
    e.aad_bytes = aad_bytes;
    for (int k = 0; k < 4; ++k) e.w[k] = le32(r.b + 4 * k);
    memcpy(out, e.w, 16);
    OPENSSL_cleanse(hb.b, 16);
    OPENSSL_cleanse(r.b, 16);
    lh_next = (lh_next + 1) % 4;
    if (lh_used < 4) ++lh_used;
}

// Te0 of the record kernels' T-table AES (public: S-box column 2, 1, 1, 3).
void te0_table(uint32_t te0[256])
{
    const uint8_t* S = sbox().s;
    for (int x = 0; x < 256; ++x) {
        const uint32_t s = S[x], s2 = gf8_mul(uint8_t(s), 2), s3 = gf8_mul(uint8_t(s), 3);
        te0[x] = s2 | (s << 8) | (s << 16) | (s3 << 24);
    }
}

// The record kernels' context image: round keys, Te0, H, the powers of H and
// the 4-bit tables of H^T, H^2T, H^UT, H^2UT.
std::vector<uint8_t> ctx_image(const uint8_t key[16], const uint8_t h[16], uint32_t npow)
{
    std::vector<uint8_t> img(sizeof(si::GcmCtx) + size_t(npow) * 16, 0);
    auto* c = reinterpret_cast<si::GcmCtx*>(img.data());
    uint8_t rk[176];
    aes_expand(key, rk);
    for (int i = 0; i < 44; ++i) {
        c->rk[i] = le32(rk + 4 * i);
        c->rk16[i] = (c->rk[i] << 16) | (c->rk[i] >> 16);
    }
    te0_table(c->te0);
    for (int k = 0; k < 4; ++k) c->h[k] = le32(h + 4 * k);
    c->npow = npow;
    Blk hb;
    memcpy(hb.b, h, 16);
    const FixedMul mh(hb);
    Blk p{};
    p.b[0] = 0x80;  // H^0 = 1
    auto* pow = reinterpret_cast<uint8_t*>(c + 1);
    for (uint32_t e = 0; e < npow; ++e) {
        memcpy(pow + 16 * size_t(e), p.b, 16);
        p = mh(p);
    }
    // Fixed multipliers of the record kernel: H^T, H^2T, H^UT, H^2UT.
    Blk ht{}, ht2{}, htu{}, htu2{};
    {
        Blk q{};
        q.b[0] = 0x80;
        for (int e = 1; e <= 2 * SI_U * SI_T; ++e) {
            q = mh(q);
            if (e == SI_T) ht = q;
            if (e == 2 * SI_T) ht2 = q;
            if (e == SI_U * SI_T) htu = q;
        }
        htu2 = q;
    }
    auto put = [](uint4* dst, const Blk& m) {
        const FixedMul mt(m);
        for (int pos = 0; pos < 32; ++pos)
            for (int v = 0; v < 16; ++v) {
                const Blk& e = mt.t[pos][v];
                dst[pos * 16 + v] = make_uint4(le32(e.b), le32(e.b + 4), le32(e.b + 8), le32(e.b + 12));
            }
    };
    put(c->gh4, ht);
    put(c->gh4b, ht2);
    put(c->gh4u, htu);
    put(c->gh4u2, htu2);
    OPENSSL_cleanse(rk, sizeof(rk));
    return img;
}

std::unique_ptr<DevCtx> build_ctx(const uint8_t key[16], const uint8_t h[16], uint32_t npow)
{
    // The host image holds the round keys: wiped once it is on the device.
    struct Image {
        std::vector<uint8_t> v;
        ~Image() { OPENSSL_cleanse(v.data(), v.size()); }
    } im{ctx_image(key, h, npow)};
    const std::vector<uint8_t>& img = im.v;
    auto out = std::make_unique<DevCtx>();
    if (hipMalloc(&out->dev, img.size()) != hipSuccess) return nullptr;
    if (hipMemcpy(out->dev, img.data(), img.size(), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    out->npow = npow;
    memcpy(out->key, key, 16);
    memcpy(out->h, h, 16);
    return out;
}

// Layout knobs (set by the tuning calls, read by every launch's layout).
std::atomic<int> g_min_rows{3};
// Cost, in rows, of a share that straddles two records (its second set of
// boundary rows, the second placement table and the two-product shares);
// MI355X, bf16 Llama-3-8B layer: 35.1 / 34.8 / 32.2 / 32.2 / 32.6 / 32.7 /
// 33.9 us per layer at 2 / 4 / 6 / 7 / 8 / 10 / 13 (int4 Qwen2.5-7B: 35.8 us
// at 4, 26.6 at 2 and 6..13; int8 and the 70B writeback flat from 6 to 10).
std::atomic<uint32_t> g_straddle_rows{6};
// Fixed cost of a record-kernel workgroup, in rows (MI355X: set-up ~3.2 us,
// placement ~1.5 us and finalisation ~0.35 us at ~1 us per row per CU), and
// whether shares of two whole records may be laid out.
uint32_t g_wg_fixed_rows = 5;
bool g_pair_records = true;

// Compute units of the current device (one record-kernel workgroup each: its
// LDS use).
uint32_t cu_count()
{
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return uint32_t(cus[dev]);
}

// The rows cover AAD || C; the length block L, the last block of the GHASH
// input, adds L * H to every record's sum (the same for the whole batch), and
// the kernel's placement exponents count one more for it.
static si::Sched make_sched_uncached(uint32_t nrec, uint64_t bytes, uint64_t aad_bytes, uint64_t cus,
                                     int min_rows, uint32_t straddle)
{
    si::Sched s{};
    s.nrec = nrec;
    s.bytes = bytes;
    s.aad_bytes = uint32_t(aad_bytes);
    s.a = uint32_t((aad_bytes + 15) / 16);
    s.n = uint32_t((bytes + 15) / 16);
    const uint64_t m = uint64_t(s.a) + s.n;
    s.rows = m ? uint32_t((m + SI_T - 1) / SI_T) : 1u;
    {
        const uint64_t pad = uint64_t(s.rows) * SI_T - m;  // blocks of row 0 before X
        s.ek_row0 = (s.a >= 1 && s.n >= 1 && pad + s.a <= SI_T - 1) ? 1u : 0u;
    }
    // W workgroups, one per CU, none with fewer than min_rows rows, and at
    // least nrec of them (rounded to whole rounds of one per CU) so that no
    // share spans more than R rows, i.e. two records at most.
    const uint64_t G = uint64_t(nrec) * s.rows;
    uint64_t w = (G + uint64_t(min_rows) - 1) / uint64_t(min_rows);
    if (w > cus) w = cus;
    if (w < nrec) w = (uint64_t(nrec) + cus - 1) / cus * cus;
    if (w > G) w = G;
    s.nwg = uint32_t(w);
    s.use_starts = 0;
    if (w > 0 && w <= SI_MAX_WG) {
        // Shares of at most T rows; a share that would end inside a record
        // continues into the next one only if it still gains rows after
        // paying the straddle cost Z (boundary rows, a second placement);
        // T is the least that fits W shares.
        const uint32_t R = s.rows, Z = straddle;
        auto lay = [&](uint32_t T, bool store) -> uint64_t {
            uint64_t n = 0, r = 0, q = 0;
            if (store) s.starts[0] = 0;
            while (r < nrec) {
                const uint64_t rem = R - q;
                if (rem >= T) {
                    q += T;
                    if (q == R) { ++r; q = 0; }
                } else if (T > Z + rem && r + 1 < nrec) {
                    q = T - Z - rem;
                    ++r;
                } else {
                    ++r;
                    q = 0;
                }
                ++n;
                if (store && n <= w) s.starts[n] = uint32_t(r * R + q);
            }
            return n;
        };
        uint32_t lo = uint32_t((G + w - 1) / w), hi = R;
        if (lo > hi) lo = hi;
        while (lo < hi) {
            const uint32_t T = lo + (hi - lo) / 2;
            if (lay(T, false) <= w) hi = T;
            else lo = T + 1;
        }
        const uint64_t n = lay(lo, true);
        for (uint64_t i = n + 1; i <= w; ++i) s.starts[i] = uint32_t(G);
        s.use_starts = 1;
        // More records than CUs: the layout above runs in rounds, each
        // workgroup paying the fixed cost.  A workgroup that takes two whole
        // records pays it once for both (one placement table serves both, as
        // each ends at row R); taken when its estimated time per CU is lower.
        if (g_pair_records && nrec > cus) {
            const uint64_t wp = (uint64_t(nrec) + 1) / 2, F = g_wg_fixed_rows;
            const uint64_t cost_rows = (w + cus - 1) / cus * (lo + F);
            const uint64_t cost_pairs = (wp + cus - 1) / cus * (2ull * R + F + 1);
            if (cost_pairs < cost_rows && wp <= SI_MAX_WG) {
                s.nwg = uint32_t(wp);
                for (uint64_t i = 0; i <= wp; ++i)
                    s.starts[i] = uint32_t((2 * i < nrec ? 2 * i : nrec) * R);
                s.pairs = 1;
            }
        }
    }
    return s;
}

// A layer's schedule depends only on its shape, the layout knobs and the
// device's CU count; a serving loop launches the same few shapes every layer,
// so each thread keeps its last few layouts (the layout search takes ~2 us
// per int4 Qwen2.5-7B layer launch and ~3 us per bf16 Llama-3-8B one on an
// x86 host core; a cached one, 0.13 us).  The cache holds no key material:
// the length block's term L * H comes from the context (DevCtx::lh_of).
// straddle: the straddle cost to lay out with, or kTunedStraddle for the
// tuning's (secure_infer_gpu_set_straddle_rows).
constexpr uint32_t kTunedStraddle = ~0u;
si::Sched make_sched(uint32_t nrec, uint64_t bytes, uint64_t aad_bytes, DevCtx& c,
                     uint32_t straddle = kTunedStraddle)
{
    struct Key {
        uint64_t bytes, aad_bytes;
        uint32_t nrec, cus, min_rows, straddle, fixed, pair;
    };
    struct Entry {
        Key k;
        si::Sched s;
    };
    constexpr int kEntries = 8;
    thread_local std::unique_ptr<Entry[]> cache;
    thread_local int used = 0, next = 0;
    Key k;
    memset(&k, 0, sizeof(k));
    k.bytes = bytes;
    k.aad_bytes = aad_bytes;
    k.nrec = nrec;
    k.cus = cu_count();
    k.min_rows = uint32_t(g_min_rows.load(std::memory_order_relaxed));
    k.straddle = straddle == kTunedStraddle ? g_straddle_rows.load(std::memory_order_relaxed) : straddle;
    k.fixed = g_wg_fixed_rows;
    k.pair = g_pair_records ? 1u : 0u;
    if (!cache) cache.reset(new Entry[kEntries]);
    si::Sched s;
    int hit = -1;
    for (int i = 0; i < used && hit < 0; ++i)
        if (!memcmp(&cache[i].k, &k, sizeof(k))) hit = i;
    if (hit >= 0) {
        s = cache[hit].s;
    } else {
        s = make_sched_uncached(nrec, bytes, aad_bytes, k.cus, int(k.min_rows), k.straddle);
        cache[next].k = k;
        cache[next].s = s;
        next = (next + 1) % kEntries;
        if (used < kEntries) ++used;
    }
    c.lh_of(bytes, aad_bytes, s.lh);
    return s;
}

uint32_t npow_for(uint64_t bytes, uint64_t aad_bytes)
{
    return uint32_t((aad_bytes + 15) / 16 + (bytes + 15) / 16 + 1 + SI_T + 16);
}

// Per-key contexts of the kernel-level entry points (keyed by key and H);
// those calls hold this lock for their whole duration.  Like every registry
// of the library it is never destroyed: its device buffers must not be freed
// by static destructors after the HIP runtime has begun to tear down.
std::mutex g_ctx_lock;
std::vector<std::unique_ptr<DevCtx>>& g_ctx_cache = *new std::vector<std::unique_ptr<DevCtx>>();

// Per-stream accumulator workspaces (and the parking area of two-record
// shares).  A launch holds its stream's workspace lock from the workspace
// lookup to the launch; launches on different streams do not contend.
struct Workspace {
    std::mutex m;
    si::RecAcc* acc = nullptr;
    size_t cap = 0;
    uint4* park = nullptr;
    size_t park_cap = 0;
};
std::mutex g_ws_lock;
std::map<std::pair<int, hipStream_t>, std::unique_ptr<Workspace>>& g_ws =
    *new std::map<std::pair<int, hipStream_t>, std::unique_ptr<Workspace>>();

Workspace* workspace_of(hipStream_t stream)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> g(g_ws_lock);
    auto& w = g_ws[std::make_pair(dev, stream)];
    if (!w) w = std::make_unique<Workspace>();
    return w.get();
}

si::RecAcc* workspace(Workspace& w, hipStream_t stream, size_t nrec)
{
    if (w.cap >= nrec) return w.acc;
    if (w.acc) {
        if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
        (void)hipFree(w.acc);
        w.acc = nullptr;
        w.cap = 0;
    }
    size_t cap = 256;
    while (cap < nrec) cap *= 2;
    if (hipMalloc(&w.acc, cap * sizeof(si::RecAcc)) != hipSuccess) return nullptr;
    if (hipMemset(w.acc, 0, cap * sizeof(si::RecAcc)) != hipSuccess) return nullptr;
    w.cap = cap;
    return w.acc;
}

// Parking area for nwg two-record workgroups (one uint4 per thread).
uint4* park_area(Workspace& w, hipStream_t stream, size_t nwg)
{
    const size_t need = nwg * SI_NT;
    if (w.park_cap >= need) return w.park;
    if (w.park) {
        if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
        (void)hipFree(w.park);
        w.park = nullptr;
        w.park_cap = 0;
    }
    if (hipMalloc(&w.park, need * sizeof(uint4)) != hipSuccess) return nullptr;
    w.park_cap = need;
    return w.park;
}

// The cached context of (key, H) from host copies, built on a miss (the
// caller holds g_ctx_lock).
DevCtx* ctx_for(const uint8_t kb[16], const uint8_t hb[16], uint32_t npow)
{
    for (auto& c : g_ctx_cache)
        if (!memcmp(c->key, kb, 16) && !memcmp(c->h, hb, 16) && c->npow >= npow) return c.get();
    auto c = build_ctx(kb, hb, npow);
    if (!c) return nullptr;
    if (g_ctx_cache.size() >= 8) {
        if (hipDeviceSynchronize() != hipSuccess) return nullptr;
        g_ctx_cache.erase(g_ctx_cache.begin());
    }
    g_ctx_cache.push_back(std::move(c));
    return g_ctx_cache.back().get();
}

// The context of a device-resident key (and H, or zeros): both read back on
// the stream first.
DevCtx* ctx_for_device_key(hipStream_t stream, const void* key, const void* h, uint32_t npow)
{
    uint8_t kb[16], hb[16] = {0};
    struct Cleanse {
        uint8_t* p;
        ~Cleanse() { OPENSSL_cleanse(p, 16); }
    } cleanse{kb};
    if (hipMemcpyAsync(kb, key, 16, hipMemcpyDeviceToHost, stream) != hipSuccess) return nullptr;
    if (h && hipMemcpyAsync(hb, h, 16, hipMemcpyDeviceToHost, stream) != hipSuccess) return nullptr;
    if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
    return ctx_for(kb, hb, npow);
}

// A context of H alone (GHASH needs no key): keyed by the all-zero key.
DevCtx* ctx_for_hash_subkey(hipStream_t stream, const void* h, uint32_t npow)
{
    uint8_t hb[16];
    static const uint8_t kZeroKey[16] = {0};
    if (hipMemcpyAsync(hb, h, 16, hipMemcpyDeviceToHost, stream) != hipSuccess) return nullptr;
    if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
    return ctx_for(kZeroKey, hb, npow);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// One record through the record kernel with context c (the caller holds
// g_ctx_lock, so c stays cached until the launch is queued).
int run_single_ctx(int mode, hipStream_t stream, DevCtx* c, void* src, void* tag, void* dst, void* status,
                   const void* ks, uint64_t bytes, const uint32_t iv[4], void* aad, uint64_t aad_bytes)
{
    Workspace* ws = workspace_of(stream);
    if (!ws) return -1;
    std::lock_guard<std::mutex> gw(ws->m);
    si::RecAcc* acc = workspace(*ws, stream, 1);
    if (!acc) return -1;
    si::RecBatch b{};
    b.single = 1;
    b.src = static_cast<const uint8_t*>(src);
    b.dst = static_cast<uint8_t*>(dst);
    b.aad = static_cast<const uint8_t*>(aad);
    b.tag = static_cast<uint8_t*>(tag);
    b.status = static_cast<uint32_t*>(status);
    b.ks = static_cast<const uint8_t*>(ks);
    for (int k = 0; k < 4; ++k) b.iv[k] = iv[k];
    const si::Sched s = make_sched(1, bytes, aad_bytes, *c);
    const bool al = aligned16(src) && (!dst || aligned16(dst)) && (!ks || aligned16(ks));
    return si::launch_gcm(mode, stream, c->dev, b, s, acc, al) == hipSuccess ? 0 : -1;
}

int run_single(int mode, hipStream_t stream, void* src, void* key, void* h, void* tag, void* dst,
               void* status, const void* ks, uint64_t bytes, const uint32_t iv[4], void* aad,
               uint64_t aad_bytes)
{
    if (bytes > SI_MAX_RECORD_BYTES) return -1;
    std::lock_guard<std::mutex> g(g_ctx_lock);
    DevCtx* c = ctx_for_device_key(stream, key, h, npow_for(bytes, aad_bytes));
    if (!c) return -1;
    return run_single_ctx(mode, stream, c, src, tag, dst, status, ks, bytes, iv, aad, aad_bytes);
}

// ---------------------------------------------------------------- control plane state

std::atomic<uint64_t> g_next_ticket{1};

struct HostRange {
    uintptr_t begin, end;
    uint32_t layer, kind;
    size_t block_bytes;
};
std::mutex g_ranges_lock;
std::vector<HostRange>& g_ranges = *new std::vector<HostRange>();

// Tickets used so far, as disjoint half-open intervals [first, last)
// (tickets are reserved in runs, so the set stays small).
std::mutex g_replay_lock;
std::map<uint64_t, uint64_t>& g_replay = *new std::map<uint64_t, uint64_t>();

bool replay_insert(uint64_t a, uint64_t b)
{
    if (a >= b) return true;
    std::lock_guard<std::mutex> g(g_replay_lock);
    auto next = g_replay.lower_bound(a);
    if (next != g_replay.end() && next->first < b) return false;
    if (next != g_replay.begin()) {
        auto prev = std::prev(next);
        if (prev->second > a) return false;
        if (prev->second == a) {  // extend the run that ends at a
            prev->second = b;
            if (next != g_replay.end() && next->first == b) {
                prev->second = next->second;
                g_replay.erase(next);
            }
            return true;
        }
    }
    if (next != g_replay.end() && next->first == b) {
        const uint64_t e = next->second;
        g_replay.erase(next);
        g_replay.emplace(a, e);
    } else {
        g_replay.emplace(a, b);
    }
    return true;
}

thread_local int64_t t_group_expected = -1;
thread_local uint32_t t_group_depth = 0;

// secure_infer_recovery_set_job_id (secure_infer.cpp:5311-5314): the job that
// records observed from now on belong to.
std::atomic<uint64_t> g_job_id{0};

struct TrackedLayer {
    hipEvent_t event;
    const uint32_t* fail_count;
    bool owned;  // event created by the library: destroyed once observed
    uint64_t job_id;
};
std::mutex g_track_lock;
std::multimap<uint32_t, TrackedLayer>& g_tracked = *new std::multimap<uint32_t, TrackedLayer>();

}  // namespace

// ---------------------------------------------------------------- sessions

struct si_session {
    std::unique_ptr<DevCtx> ctx;
    uint32_t salt_word;
    uint64_t session_nonce;
    uint64_t max_record_bytes;
    std::atomic<uint32_t> holds{0};  // pending launches / jobs naming it (si_host.cpp)
};

extern "C" {

const char* secure_infer_gpu_version(void)
{
    return "secure_infer_amd 0.1 (gfx950, AES-128-GCM T-table/LDS, 4-bit GHASH tables)";
}

int secure_infer_gpu_session_create(const uint8_t key[16], const uint8_t iv_salt[4],
                                    uint64_t session_nonce, uint64_t max_record_bytes,
                                    si_session** out)
{
    if (!key || !iv_salt || !out || max_record_bytes == 0 || max_record_bytes > SI_MAX_RECORD_BYTES)
        return -1;
    uint8_t rk[176], h[16], zero[16] = {0};
    aes_expand(key, rk);
    aes_encrypt(rk, zero, h);
    OPENSSL_cleanse(rk, sizeof(rk));
    auto s = std::make_unique<si_session>();
    s->ctx = build_ctx(key, h, npow_for(max_record_bytes, 64));
    if (!s->ctx) return -1;
    s->salt_word = be32(iv_salt);
    s->session_nonce = session_nonce;
    s->max_record_bytes = max_record_bytes;
    *out = s.release();
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------- session key agreement

namespace {

// Host half of the agreement through OpenSSL (the reference uses Monocypher's
// crypto_x25519 / crypto_blake2b_keyed, secure_infer.cpp:466-499).
bool x25519_public(const uint8_t secret[32], uint8_t out[32])
{
    EVP_PKEY* k = EVP_PKEY_new_raw_private_key(EVP_PKEY_X25519, nullptr, secret, 32);
    size_t len = 32;
    const bool ok = k && EVP_PKEY_get_raw_public_key(k, out, &len) == 1 && len == 32;
    EVP_PKEY_free(k);
    return ok;
}

bool x25519_shared(const uint8_t secret[32], const uint8_t peer[32], uint8_t out[32])
{
    EVP_PKEY* k = EVP_PKEY_new_raw_private_key(EVP_PKEY_X25519, nullptr, secret, 32);
    EVP_PKEY* p = EVP_PKEY_new_raw_public_key(EVP_PKEY_X25519, nullptr, peer, 32);
    EVP_PKEY_CTX* c = k ? EVP_PKEY_CTX_new(k, nullptr) : nullptr;
    size_t len = 32;
    const bool ok = c && p && EVP_PKEY_derive_init(c) == 1 && EVP_PKEY_derive_set_peer(c, p) == 1 &&
                    EVP_PKEY_derive(c, out, &len) == 1 && len == 32;
    EVP_PKEY_CTX_free(c);
    EVP_PKEY_free(p);
    EVP_PKEY_free(k);
    return ok;
}

// BLAKE2b keyed by `key`, `out_len` bytes, over the concatenation of parts.
bool blake2b_keyed(const uint8_t* key, size_t key_len, std::initializer_list<std::pair<const void*, size_t>> parts,
                   uint8_t* out, size_t out_len)
{
    EVP_MAC* mac = EVP_MAC_fetch(nullptr, "BLAKE2BMAC", nullptr);
    EVP_MAC_CTX* c = mac ? EVP_MAC_CTX_new(mac) : nullptr;
    OSSL_PARAM params[2] = {OSSL_PARAM_construct_size_t(OSSL_MAC_PARAM_SIZE, &out_len), OSSL_PARAM_construct_end()};
    bool ok = c && EVP_MAC_init(c, key, key_len, params) == 1;
    for (const auto& part : parts) ok = ok && EVP_MAC_update(c, static_cast<const uint8_t*>(part.first), part.second) == 1;
    size_t len = 0;
    ok = ok && EVP_MAC_final(c, out, &len, out_len) == 1 && len == out_len;
    EVP_MAC_CTX_free(c);
    EVP_MAC_free(mac);
    return ok;
}

// Test-only one-shot fault for the next agreement (secure_infer_test_tamper_agree).
std::atomic<uint32_t> g_tamper_agree{0};

const char kAgreeInfo[] = "SecureInfer X25519 BLAKE2b test v1";
const char kSaltInfo[] = "SecureInfer IV salt v1";

// Builds the record kernels' context on the device from a device-resident
// key (the key's bytes never leave the device).
std::unique_ptr<DevCtx> build_ctx_on_device(hipStream_t stream, const uint8_t* dev_key, uint32_t npow)
{
    uint32_t te0[256];
    te0_table(te0);
    uint32_t* d_te0 = nullptr;
    auto out = std::make_unique<DevCtx>();
    const size_t bytes = sizeof(si::GcmCtx) + size_t(npow) * 16;
    bool ok = hipMalloc(reinterpret_cast<void**>(&out->dev), bytes) == hipSuccess &&
              hipMalloc(reinterpret_cast<void**>(&d_te0), sizeof(te0)) == hipSuccess &&
              hipMemcpyAsync(d_te0, te0, sizeof(te0), hipMemcpyHostToDevice, stream) == hipSuccess &&
              si::launch_ctx_build(stream, dev_key, d_te0, out->dev, npow) == hipSuccess &&
              hipStreamSynchronize(stream) == hipSuccess;
    if (d_te0) (void)hipFree(d_te0);
    if (!ok) return nullptr;
    out->npow = npow;
    return out;
}

// Address of a field of a device-resident struct.
uint8_t* field(void* dev_struct, size_t offset) { return static_cast<uint8_t*>(dev_struct) + offset; }

// Device buffers of one agreement, freed on exit.  The key and the entropy
// pool (with the seed, the pool determines the device's X25519 secret) are
// zeroed first.
struct AgreeBufs {
    hipStream_t stream = nullptr;
    si::AgreeIo* io = nullptr;
    uint8_t* key = nullptr;
    uint32_t* pool = nullptr;
    uint32_t* counter = nullptr;
    ~AgreeBufs()
    {
        if (stream) {
            if (key) (void)si::launch_zero_bytes(stream, key, 16);
            if (pool) (void)si::launch_zero_bytes(stream, reinterpret_cast<uint8_t*>(pool), SI_AGREE_POOL_WORDS * 4u);
            (void)hipStreamSynchronize(stream);
        }
        for (void* p : {static_cast<void*>(io), static_cast<void*>(key), static_cast<void*>(pool),
                        static_cast<void*>(counter)})
            if (p) (void)hipFree(p);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

}  // namespace

extern "C" {

int secure_infer_gpu_session_agree(uint64_t session_nonce, uint64_t max_record_bytes, si_session** out)
{
    if (!out || max_record_bytes == 0 || max_record_bytes > SI_MAX_RECORD_BYTES) return -1;
    uint8_t secret[32], host_public[32], shared[32], key[16], expected[32], salt[4], h[16], rk[176], zero[16] = {0};
    si::AgreeIo io{};
    si::AgreeSeed seed{};
    int rc = -1;
    std::unique_ptr<si_session> s;
    {
        AgreeBufs b;
        if (RAND_bytes(secret, 32) != 1 || RAND_bytes(io.challenge, 32) != 1 || RAND_bytes(seed.b, 32) != 1 ||
            !x25519_public(secret, host_public))
            goto done;
        const uint32_t fault = g_tamper_agree.exchange(0);
        memcpy(io.host_public, host_public, 32);
        if (fault == 2) memset(io.host_public, 0, 32);
        io.status = -1;
        // A private stream, as the reference's setup stream: nothing the
        // caller has queued is waited for.
        if (hipStreamCreateWithFlags(&b.stream, hipStreamNonBlocking) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&b.io), sizeof(si::AgreeIo)) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&b.key), 16) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&b.pool), SI_AGREE_POOL_WORDS * 4) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&b.counter), 4) != hipSuccess ||
            hipMemcpyAsync(b.io, &io, sizeof(io), hipMemcpyHostToDevice, b.stream) != hipSuccess ||
            si::launch_agree(b.stream, field(b.io, offsetof(si::AgreeIo, host_public)),
                             field(b.io, offsetof(si::AgreeIo, challenge)), seed, b.pool, b.counter, b.key,
                             field(b.io, offsetof(si::AgreeIo, device_public)),
                             field(b.io, offsetof(si::AgreeIo, proof)),
                             reinterpret_cast<int32_t*>(field(b.io, offsetof(si::AgreeIo, status)))) != hipSuccess ||
            hipMemcpyAsync(&io, b.io, sizeof(io), hipMemcpyDeviceToHost, b.stream) != hipSuccess ||
            hipStreamSynchronize(b.stream) != hipSuccess || io.status != 0)
            goto done;
        if (fault == 1) io.proof[0] ^= 0x01;
        {
            uint8_t nz = 0;
            if (!x25519_shared(secret, io.device_public, shared)) goto done;
            for (uint8_t v : shared) nz |= v;
            if (!nz) goto done;
        }
        if (!blake2b_keyed(shared, 32,
                           {{kAgreeInfo, sizeof(kAgreeInfo) - 1}, {host_public, 32}, {io.device_public, 32},
                            {io.challenge, 32}},
                           key, 16) ||
            !blake2b_keyed(key, 16, {{io.challenge, 32}}, expected, 32) ||
            !blake2b_keyed(shared, 32, {{kSaltInfo, sizeof(kSaltInfo) - 1}}, salt, 4) ||
            CRYPTO_memcmp(expected, io.proof, 32) != 0)
            goto done;
        s = std::make_unique<si_session>();
        s->ctx = build_ctx_on_device(b.stream, b.key, npow_for(max_record_bytes, 64));
        if (!s->ctx) goto done;
        // The host keeps its own copy of the agreed key for OpenSSL.
        aes_expand(key, rk);
        aes_encrypt(rk, zero, h);
        memcpy(s->ctx->key, key, 16);
        memcpy(s->ctx->h, h, 16);
        s->salt_word = be32(salt);
        s->session_nonce = session_nonce;
        s->max_record_bytes = max_record_bytes;
        rc = 0;
    }
done:
    OPENSSL_cleanse(secret, sizeof(secret));
    OPENSSL_cleanse(seed.b, sizeof(seed.b));
    OPENSSL_cleanse(shared, sizeof(shared));
    OPENSSL_cleanse(key, sizeof(key));
    OPENSSL_cleanse(rk, sizeof(rk));
    if (rc != 0) return -1;
    *out = s.release();
    return 0;
}

int secure_infer_test_tamper_agree(uint32_t mode)
{
    if (mode > 2) return -1;
    g_tamper_agree.store(mode);
    return 0;
}

int64_t secure_infer_test_context_image(const uint8_t key[16], uint64_t max_record_bytes, int on_device, void* out,
                                        uint64_t cap)
{
    if (!key || max_record_bytes == 0 || max_record_bytes > SI_MAX_RECORD_BYTES) return -1;
    const uint32_t npow = npow_for(max_record_bytes, 64);
    const uint64_t bytes = sizeof(si::GcmCtx) + uint64_t(npow) * 16;
    if (!out) return int64_t(bytes);
    if (cap < bytes) return -1;
    if (!on_device) {
        uint8_t rk[176], h[16], zero[16] = {0};
        aes_expand(key, rk);
        aes_encrypt(rk, zero, h);
        const std::vector<uint8_t> img = ctx_image(key, h, npow);
        memcpy(out, img.data(), bytes);
        return int64_t(bytes);
    }
    hipStream_t st = nullptr;
    uint8_t* d_key = nullptr;
    bool ok = hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess &&
              hipMalloc(reinterpret_cast<void**>(&d_key), 16) == hipSuccess &&
              hipMemcpyAsync(d_key, key, 16, hipMemcpyHostToDevice, st) == hipSuccess;
    std::unique_ptr<DevCtx> c = ok ? build_ctx_on_device(st, d_key, npow) : nullptr;
    ok = c && hipMemcpy(out, c->dev, bytes, hipMemcpyDeviceToHost) == hipSuccess;
    if (d_key) (void)hipFree(d_key);
    if (st) (void)hipStreamDestroy(st);
    return ok ? int64_t(bytes) : -1;
}

int secure_infer_test_x25519(const uint8_t scalar[32], const uint8_t u[32], uint8_t out[32])
{
    if (!scalar || !u || !out) return -1;
    uint8_t* d = nullptr;
    bool ok = hipMalloc(reinterpret_cast<void**>(&d), 96) == hipSuccess &&
              hipMemcpy(d, scalar, 32, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(d + 32, u, 32, hipMemcpyHostToDevice) == hipSuccess &&
              si::launch_x25519_test(nullptr, d, d + 32, d + 64) == hipSuccess &&
              hipMemcpy(out, d + 64, 32, hipMemcpyDeviceToHost) == hipSuccess;
    if (d) (void)hipFree(d);
    return ok ? 0 : -1;
}

int secure_infer_test_blake2b(const uint8_t* key, uint32_t key_len, const uint8_t* msg, uint64_t msg_len,
                              uint8_t* out, uint32_t out_len)
{
    if ((key_len && !key) || key_len > 64 || (msg_len && !msg) || !out || out_len == 0 || out_len > 64) return -1;
    uint8_t* d = nullptr;
    const uint64_t n = 64 + 64 + msg_len + 1;
    bool ok = hipMalloc(reinterpret_cast<void**>(&d), n) == hipSuccess &&
              (key_len == 0 || hipMemcpy(d, key, key_len, hipMemcpyHostToDevice) == hipSuccess) &&
              (msg_len == 0 || hipMemcpy(d + 128, msg, msg_len, hipMemcpyHostToDevice) == hipSuccess) &&
              si::launch_blake2b_test(nullptr, d, key_len, d + 128, msg_len, d + 64, out_len) == hipSuccess &&
              hipMemcpy(out, d + 64, out_len, hipMemcpyDeviceToHost) == hipSuccess;
    if (d) (void)hipFree(d);
    return ok ? 0 : -1;
}

int secure_infer_gpu_session_destroy(si_session* s)
{
    if (!s) return -1;
    if (!si_internal::forget_session(s)) {
        fprintf(stderr, "[secure_infer] session_destroy: another thread still has swaps of this session "
                        "that were not issued (an open layer group or D2H batch); end them first\n");
        return -1;
    }
    (void)hipDeviceSynchronize();
    delete s;
    return 0;
}

int secure_infer_gpu_session_hash_subkey(const si_session* s, uint8_t out[16])
{
    if (!s || !out) return -1;
    memcpy(out, s->ctx->h, 16);
    return 0;
}

uint64_t secure_infer_codec_width(uint32_t bits, uint32_t heads, uint32_t head_dim)
{
    const uint64_t qb = 128ull * heads * head_dim * bits / 8;
    const uint64_t sb = 2ull * heads * head_dim * 4;
    return (qb + 2 * sb + 16 + 15) / 16 * 16;
}

uint64_t secure_infer_wire_stride(uint64_t bytes)
{
    return ((bytes + 31) & ~uint64_t(31)) + 96;
}

static int layer_common(const si_session* s, uint64_t bytes, uint32_t nrec, uint32_t n_k,
                        uint64_t nslots, uint64_t wire_stride, const void* wire, const int64_t* slots,
                        uint32_t codec, uint32_t heads, uint32_t dim, const void* staging,
                        uint64_t slot_bytes)
{
    if (!s || !wire || !slots || nrec == 0 || n_k > nrec || bytes == 0) return -1;
    if (nslots == 0 || bytes > SI_MAX_RECORD_BYTES) return -1;
    if (bytes > s->max_record_bytes) return -1;
    if (wire_stride < secure_infer_wire_stride(bytes) || (wire_stride & 15)) return -1;
    if (!aligned16(wire)) return -1;
    if (codec != SI_CODEC_NONE && codec != SI_CODEC_INT8 && codec != SI_CODEC_INT4) return -1;
    if (codec != SI_CODEC_NONE) {
        if (!staging || !aligned16(staging) || heads == 0 || dim == 0 || dim % 64) return -1;
        if (bytes != secure_infer_codec_width(codec, heads, dim)) return -1;
        if (slot_bytes < 128ull * heads * dim * 2) return -1;
    } else if (slot_bytes < bytes) {
        return -1;
    }
    return 0;
}

static void fill_layer_ivs(const si_session* s, si::RecBatch& b, const uint32_t* ivs, uint64_t ticket_base)
{
    b.ivs = ivs;
    b.iv[0] = s->salt_word;
    b.iv[3] = 2;
    b.nonce_base = s->session_nonce + ticket_base;
}

// Checks of a reload descriptor shared by both reload entry points (the
// codec staging buffer is checked by the caller: the allocation-free entry
// point brings its own).
static int reload_checks(const si_session* s, const si_reload_desc* d, const void* staging)
{
    if (!d) return -1;
    if (layer_common(s, d->bytes, d->nrec, d->n_k, d->nslots, d->wire_stride, d->wire, d->slots, d->codec_bits,
                     d->heads, d->head_dim, staging, d->slot_bytes))
        return -1;
    if (!d->cache_k && d->n_k) return -1;
    if (!d->cache_v && d->n_k < d->nrec) return -1;
    if (!d->iv_words && d->ticket_base == 0) return -1;
    if (d->flags & ~uint32_t(SI_RELOAD_VERIFY_BEFORE_RELEASE)) return -1;
    return 0;
}

// Events armed by secure_infer_gpu_time_next_layer for the calling thread's
// next layer launch (one shot).
thread_local si::LaunchEvents t_layer_events;
// Clock probes armed by secure_infer_gpu_clock_next_layers for the calling
// thread's next layer launches, one per layer in launch order; each keeps the
// words its launch used and its overflow flag for
// secure_infer_gpu_clock_layers_used.
thread_local std::vector<si::ClockProbe> t_clock_layers;
thread_local size_t t_clock_next = 0;

static si::LaunchEvents take_layer_events()
{
    si::LaunchEvents ev = t_layer_events;
    t_layer_events = si::LaunchEvents();
    if (t_clock_next < t_clock_layers.size()) ev.clock = &t_clock_layers[t_clock_next++];
    return ev;
}

// Test hook (secure_infer_test_strict_phases): the calling thread's next
// verify-before-release reload stops after its first `n` launches (0: all).
thread_local int t_strict_phases = 0;

static int take_strict_phases()
{
    const int n = t_strict_phases;
    t_strict_phases = 0;
    return n;
}

// The verify / decrypt launch and, with a codec, the dequantise-scatter
// launch of one reload layer, given its accumulators, schedule (with its
// parking area) and staging.
static int reload_launch(hipStream_t stream, si_session* s, const si_reload_desc* d, si::RecAcc* acc,
                         const si::Sched& sc, uint8_t* staging, const uint32_t* gate = nullptr)
{
    si::RecBatch b{};
    b.single = 0;
    b.encrypt = 0;
    b.wire = static_cast<const uint8_t*>(d->wire);
    b.wire_stride = d->wire_stride;
    b.tag_off = (d->bytes + 31) & ~uint64_t(31);
    b.status_off = b.tag_off + 16;
    b.aad_off = b.tag_off + 32;
    b.cache[0] = static_cast<uint8_t*>(d->cache_k);
    b.cache[1] = static_cast<uint8_t*>(d->cache_v);
    b.slot_bytes = d->slot_bytes;
    b.slots = d->slots;
    b.nslots = int64_t(d->nslots);
    b.n_k = d->n_k;
    fill_layer_ivs(s, b, d->iv_words, d->ticket_base);
    b.fail_count = d->fail_count;
    const bool codec = d->codec_bits != SI_CODEC_NONE;
    if (codec) {
        b.staging = staging;
        b.staging_stride = (d->bytes + 31) & ~uint64_t(31);
    }
    const bool al = aligned16(d->cache_k) && aligned16(d->cache_v) && (d->slot_bytes % 16 == 0);
    si::Sched sc2 = sc;
    sc2.status_out = d->status_out;
    sc2.gate = gate;
    const bool strict = (d->flags & SI_RELOAD_VERIFY_BEFORE_RELEASE) != 0;
    const int phases = take_strict_phases();
    // A timed layer: start at the first kernel, stop at the layer's last kernel.
    const si::LaunchEvents ev = take_layer_events();
    si::LaunchEvents ev_rec = ev, ev_rel, ev_dq;
    ev_rel.clock = ev_dq.clock = ev.clock;
    if (strict) {
        ev_rec.stop = nullptr;
        ev_rel.stop = codec ? nullptr : ev.stop;
    } else if (codec) {
        ev_rec.stop = nullptr;
    }
    if (codec) ev_dq.stop = ev.stop;
    if (strict) {
        // Tags and statuses first (nothing else written), then the release.
        // The verification hashes without decrypting, so its rows cost
        // about a third of a decrypting row's time while a straddling
        // share's second start costs the same: it is laid out without
        // straddling shares (MI355X, bf16 Llama-3-8B layer 44.7 -> 41.6 us
        // per layer, ABBA on one GPU).  A layout that pairs records keeps
        // the caller's, whose parking area is sized for it.
        si::Sched sv = sc2;
        if (!sc.pairs) {
            si::Sched t = make_sched(d->nrec, d->bytes, 64, *s->ctx, 256u);
            if (!t.pairs) {
                t.status_out = d->status_out;
                t.gate = gate;
                sv = t;
            }
        }
        if (si::launch_gcm(2, stream, s->ctx->dev, b, sv, acc, al, ev_rec) != hipSuccess) return -1;
        if (phases == 1) return 0;
        if (si::launch_release(stream, s->ctx->dev, b, d->nrec, d->bytes, al || codec, gate, cu_count(), ev_rel) != hipSuccess)
            return -1;
    } else if (si::launch_gcm(0, stream, s->ctx->dev, b, sc2, acc, al, ev_rec) != hipSuccess) {
        return -1;
    }
    if (codec) {
        si::CodecBatch cb{};
        cb.nrec = d->nrec;
        cb.n_k = d->n_k;
        cb.bits = d->codec_bits;
        cb.heads = d->heads;
        cb.dim = d->head_dim;
        cb.layer = d->layer;
        cb.cache[0] = static_cast<uint8_t*>(d->cache_k);
        cb.cache[1] = static_cast<uint8_t*>(d->cache_v);
        cb.slot_bytes = d->slot_bytes;
        cb.slots = d->slots;
        cb.nslots = int64_t(d->nslots);
        cb.staging = staging;
        cb.staging_stride = b.staging_stride;
        cb.qbytes = 128ull * d->heads * d->head_dim * d->codec_bits / 8;
        cb.sbytes = 2ull * d->heads * d->head_dim * 4;
        cb.width = d->bytes;
        cb.gate = gate;
        if (si::launch_dequant_scatter(stream, cb, ev_dq) != hipSuccess) return -1;
    }
    return 0;
}

int secure_infer_gpu_reload_layer(hipStream_t stream, si_session* s, const si_reload_desc* d)
{
    if (!d || reload_checks(s, d, d->staging)) return -1;
    Workspace* ws = workspace_of(stream);
    if (!ws) return -1;
    std::lock_guard<std::mutex> g(ws->m);
    si::RecAcc* acc = workspace(*ws, stream, d->nrec);
    if (!acc) return -1;
    si::Sched sc = make_sched(d->nrec, d->bytes, 64, *s->ctx);
    if (sc.pairs && !(sc.park = park_area(*ws, stream, sc.nwg))) return -1;
    return reload_launch(stream, s, d, acc, sc, static_cast<uint8_t*>(d->staging));
}

int secure_infer_gpu_reload_layer_noalloc(hipStream_t stream, si_session* s, const si_reload_desc* d)
{
    if (!d) return -1;
    if (d->staging) {
        fprintf(stderr, "[secure_infer] reload_layer_noalloc: staging must be NULL (the library's scratch "
                        "holds it)\n");
        return -1;
    }
    const bool codec = d->codec_bits != SI_CODEC_NONE;
    // layer_common wants a staging pointer for a codec; the scratch's is
    // only known once the request fits, so check with a stand-in first.
    if (reload_checks(s, d, codec ? reinterpret_cast<const void*>(uintptr_t(256)) : nullptr)) return -1;
    si::Sched sc = make_sched(d->nrec, d->bytes, 64, *s->ctx);
    const uint64_t park_bytes = sc.pairs ? (uint64_t(sc.nwg) * SI_NT * sizeof(uint4) + 255) / 256 * 256 : 0;
    const uint64_t stage_bytes = codec ? uint64_t(d->nrec) * ((d->bytes + 31) & ~uint64_t(31)) : 0;
    const uint64_t need = SI_NOALLOC_CTRL_BYTES + SI_NOALLOC_ACC_BYTES + park_bytes + stage_bytes;
    if (d->nrec > SI_NOALLOC_MAX_RECORDS || need > SI_NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr,
                "[secure_infer] reload_layer_noalloc: %u records of %llu B need %llu B of scratch "
                "(at most %u records and %llu B); use secure_infer_gpu_reload_layer\n",
                d->nrec, static_cast<unsigned long long>(d->bytes), static_cast<unsigned long long>(need),
                SI_NOALLOC_MAX_RECORDS, static_cast<unsigned long long>(SI_NOALLOC_SCRATCH_BYTES));
        return -1;
    }
    uint8_t* base = si::noalloc_scratch(stream);
    if (!base) return -1;
    uint32_t* ctrl = reinterpret_cast<uint32_t*>(base);
    si::RecAcc* acc = reinterpret_cast<si::RecAcc*>(base + SI_NOALLOC_CTRL_BYTES);
    uint8_t* after_acc = base + SI_NOALLOC_CTRL_BYTES + SI_NOALLOC_ACC_BYTES;
    if (sc.pairs) sc.park = reinterpret_cast<uint4*>(after_acc);
    uint8_t* staging = codec ? after_acc + park_bytes : nullptr;
    // The call's lock cell: bytes 4..7 of record 0's status slot (its own
    // memory; the kernels write only the status word, bytes 0..3).
    uint8_t* wire = static_cast<uint8_t*>(const_cast<void*>(d->wire));
    const uint64_t status_off = ((d->bytes + 31) & ~uint64_t(31)) + 16;
    uint32_t* cell = reinterpret_cast<uint32_t*>(wire + status_off + 4);
    if (si::launch_noalloc_acquire(stream, ctrl, cell) != hipSuccess) return -1;
    const int rc = reload_launch(stream, s, d, acc, sc, staging, cell);
    // The finishing kernel runs even after a failed launch: it returns the
    // owner word (or fails the records closed), so no call keeps the scratch.
    si::NoallocFinish f{};
    f.ctrl = ctrl;
    f.cell = cell;
    f.wire = wire;
    f.wire_stride = d->wire_stride;
    f.status_off = status_off;
    f.cache[0] = static_cast<uint8_t*>(d->cache_k);
    f.cache[1] = static_cast<uint8_t*>(d->cache_v);
    f.slot_bytes = d->slot_bytes;
    f.out_bytes = codec ? 128ull * d->heads * d->head_dim * 2 : d->bytes;
    f.slots = d->slots;
    f.nslots = int64_t(d->nslots);
    f.nrec = d->nrec;
    f.n_k = d->n_k;
    f.status_out = d->status_out;
    f.fail_count = d->fail_count;
    if (si::launch_noalloc_finish(stream, f) != hipSuccess) return -1;
    return rc;
}

int secure_infer_gpu_time_next_layer(hipEvent_t start, hipEvent_t stop)
{
    if (!start && !stop) return -1;
    t_layer_events.start = start;
    t_layer_events.stop = stop;
    return 0;
}

int secure_infer_gpu_clock_next_layers(uint64_t* stamps, uint64_t words_per_layer, uint32_t layers)
{
    if (!stamps || words_per_layer == 0 || layers == 0 || words_per_layer > UINT64_MAX / layers) return -1;
    t_clock_layers.assign(layers, si::ClockProbe());
    for (uint32_t l = 0; l < layers; ++l) {
        t_clock_layers[l].stamps = stamps + uint64_t(l) * words_per_layer;
        t_clock_layers[l].words = words_per_layer;
    }
    t_clock_next = 0;
    return 0;
}

int secure_infer_gpu_clock_layers_used(uint64_t* words_used, uint32_t layers)
{
    if (layers == 0 || layers > t_clock_next) return -1;
    for (uint32_t l = 0; l < layers; ++l) {
        if (t_clock_layers[l].overflow) return -1;
        if (words_used) words_used[l] = t_clock_layers[l].used;
    }
    return 0;
}

int secure_infer_gpu_clock_rate_khz(uint64_t* khz)
{
    int dev = 0, rate = 0;
    if (!khz || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev) != hipSuccess || rate <= 0)
        return -1;
    *khz = uint64_t(rate);
    return 0;
}

int secure_infer_test_strict_phases(int n)
{
    if (n < 0) return -1;
    t_strict_phases = n;
    return 0;
}

int secure_infer_test_noalloc_hold(hipStream_t stream, int hold)
{
    uint8_t* base = si::noalloc_scratch(stream);
    if (!base) return -1;
    return si::launch_noalloc_test_hold(stream, reinterpret_cast<uint32_t*>(base), hold) == hipSuccess ? 0 : -1;
}

int secure_infer_gpu_writeback_layer(hipStream_t stream, si_session* s, const si_writeback_desc* d)
{
    if (!d) return -1;
    if (layer_common(s, d->bytes, d->nrec, d->n_k, d->nslots, d->wire_stride, d->wire, d->slots, d->codec_bits,
                     d->heads, d->head_dim, d->staging, d->slot_bytes))
        return -1;
    if (!d->cache_k && d->n_k) return -1;
    if (!d->cache_v && d->n_k < d->nrec) return -1;
    if (!d->iv_words && d->ticket_base == 0) return -1;
    Workspace* ws = workspace_of(stream);
    if (!ws) return -1;
    std::lock_guard<std::mutex> g(ws->m);
    si::RecAcc* acc = workspace(*ws, stream, d->nrec);
    if (!acc) return -1;
    const bool codec = d->codec_bits != SI_CODEC_NONE;
    si::RecBatch b{};
    b.single = 0;
    b.encrypt = 1;
    b.wire = static_cast<const uint8_t*>(d->wire);
    b.wire_stride = d->wire_stride;
    b.tag_off = (d->bytes + 31) & ~uint64_t(31);
    b.status_off = b.tag_off + 16;
    b.aad_off = b.tag_off + 32;
    b.cache[0] = static_cast<uint8_t*>(const_cast<void*>(d->cache_k));
    b.cache[1] = static_cast<uint8_t*>(const_cast<void*>(d->cache_v));
    b.slot_bytes = d->slot_bytes;
    b.slots = d->slots;
    b.nslots = int64_t(d->nslots);
    b.n_k = d->n_k;
    b.fail_count = d->fail_count;
    fill_layer_ivs(s, b, d->iv_words, d->ticket_base);
    // A timed layer: start at the layer's first kernel, stop at the record kernel.
    const si::LaunchEvents ev = take_layer_events();
    si::LaunchEvents ev_q, ev_rec = ev;
    ev_q.clock = ev.clock;
    if (codec) {
        ev_q.start = ev.start;
        ev_rec.start = nullptr;
    }
    if (codec) {
        b.staging = static_cast<uint8_t*>(d->staging);
        b.staging_stride = (d->bytes + 31) & ~uint64_t(31);
        si::CodecBatch cb{};
        cb.nrec = d->nrec;
        cb.n_k = d->n_k;
        cb.bits = d->codec_bits;
        cb.heads = d->heads;
        cb.dim = d->head_dim;
        cb.layer = d->layer;
        cb.cache[0] = b.cache[0];
        cb.cache[1] = b.cache[1];
        cb.slot_bytes = d->slot_bytes;
        cb.slots = d->slots;
        cb.nslots = int64_t(d->nslots);
        cb.staging = b.staging;
        cb.staging_stride = b.staging_stride;
        cb.qbytes = 128ull * d->heads * d->head_dim * d->codec_bits / 8;
        cb.sbytes = 2ull * d->heads * d->head_dim * 4;
        cb.width = d->bytes;
        if (si::launch_gather_quant(stream, cb, ev_q) != hipSuccess) return -1;
    }
    si::Sched sc = make_sched(d->nrec, d->bytes, 64, *s->ctx);
    if (sc.pairs && !(sc.park = park_area(*ws, stream, sc.nwg))) return -1;
    const bool al = aligned16(d->cache_k) && aligned16(d->cache_v) && (d->slot_bytes % 16 == 0);
    return si::launch_gcm(1, stream, s->ctx->dev, b, sc, acc, al, ev_rec) == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------- kernel-level mirrors

int secure_infer_gpu_gcm_decrypt_verify_aad_do(hipStream_t stream, void* ciphertext, void* key,
                                               void* hash_subkey, void* expected_tag,
                                               void* plaintext_output, void* status_output,
                                               uint64_t bytes, uint32_t iv0, uint32_t iv1,
                                               uint32_t iv2, uint32_t iv3, void* aad,
                                               uint64_t aad_bytes)
{
    if (!ciphertext || !key || !hash_subkey || !expected_tag || !plaintext_output || !status_output ||
        bytes == 0 || (aad_bytes != 0 && !aad))
        return -1;
    const uint32_t iv[4] = {iv0, iv1, iv2, iv3};
    return run_single(0, stream, ciphertext, key, hash_subkey, expected_tag, plaintext_output,
                      status_output, nullptr, bytes, iv, aad, aad_bytes);
}

int secure_infer_gpu_gcm_decrypt_verify_do(hipStream_t stream, void* ciphertext, void* key,
                                           void* hash_subkey, void* expected_tag,
                                           void* plaintext_output, void* status_output,
                                           uint64_t bytes, uint32_t iv0, uint32_t iv1,
                                           uint32_t iv2, uint32_t iv3)
{
    return secure_infer_gpu_gcm_decrypt_verify_aad_do(stream, ciphertext, key, hash_subkey,
                                                      expected_tag, plaintext_output,
                                                      status_output, bytes, iv0, iv1, iv2, iv3,
                                                      nullptr, 0);
}

int secure_infer_gpu_gcm_encrypt_tag_do(hipStream_t stream, void* plaintext, void* key,
                                        void* hash_subkey, void* ciphertext_output,
                                        void* tag_output, uint64_t bytes, uint32_t iv0,
                                        uint32_t iv1, uint32_t iv2, uint32_t iv3, void* aad,
                                        uint64_t aad_bytes)
{
    if (!plaintext || !key || !hash_subkey || !ciphertext_output || !tag_output || bytes == 0 ||
        (aad_bytes != 0 && !aad))
        return -1;
    const uint32_t iv[4] = {iv0, iv1, iv2, iv3};
    return run_single(1, stream, plaintext, key, hash_subkey, tag_output, ciphertext_output,
                      nullptr, nullptr, bytes, iv, aad, aad_bytes);
}

int secure_infer_gpu_gcm_verify_only_aad_do(hipStream_t stream, void* ciphertext, void* key,
                                            void* hash_subkey, void* expected_tag,
                                            void* status_output, uint64_t bytes, uint32_t iv0,
                                            uint32_t iv1, uint32_t iv2, uint32_t iv3, void* aad,
                                            uint64_t aad_bytes)
{
    if (!ciphertext || !key || !hash_subkey || !expected_tag || !status_output || bytes == 0 ||
        (aad_bytes != 0 && !aad))
        return -1;
    const uint32_t iv[4] = {iv0, iv1, iv2, iv3};
    return run_single(2, stream, ciphertext, key, hash_subkey, expected_tag, nullptr,
                      status_output, nullptr, bytes, iv, aad, aad_bytes);
}

int secure_infer_gpu_gcm_verify_xor_aad_do(hipStream_t stream, void* ciphertext, void* key,
                                           void* hash_subkey, void* expected_tag, void* keystream,
                                           void* plaintext_output, void* status_output,
                                           uint64_t bytes, uint32_t iv0, uint32_t iv1,
                                           uint32_t iv2, uint32_t iv3, void* aad,
                                           uint64_t aad_bytes)
{
    if (!ciphertext || !key || !hash_subkey || !expected_tag || !keystream || !plaintext_output ||
        !status_output || bytes == 0 || (aad_bytes != 0 && !aad))
        return -1;
    const uint32_t iv[4] = {iv0, iv1, iv2, iv3};
    return run_single(3, stream, ciphertext, key, hash_subkey, expected_tag, plaintext_output,
                      status_output, keystream, bytes, iv, aad, aad_bytes);
}

static int run_ctr(hipStream_t stream, const void* in, void* key, void* out, uint64_t bytes,
                   const uint32_t iv[4])
{
    std::lock_guard<std::mutex> g(g_ctx_lock);
    DevCtx* c = ctx_for_device_key(stream, key, nullptr, 1);
    if (!c) return -1;
    return si::launch_ctr(stream, c->dev, static_cast<const uint8_t*>(in), static_cast<uint8_t*>(out),
                          bytes, iv) == hipSuccess ? 0 : -1;
}

int secure_infer_gpu_aes_ctr_do(hipStream_t stream, void* input, void* key, void* output,
                                uint64_t bytes, uint32_t iv0, uint32_t iv1, uint32_t iv2,
                                uint32_t iv3)
{
    if (!input || !key || !output || bytes == 0) return -1;
    const uint32_t iv[4] = {iv0, iv1, iv2, iv3};
    return run_ctr(stream, input, key, output, bytes, iv);
}

int secure_infer_gpu_keystream_do(hipStream_t stream, void* key, void* output, uint64_t bytes,
                                  uint32_t iv0, uint32_t iv1, uint32_t iv2, uint32_t iv3)
{
    if (!key || !output || bytes == 0) return -1;
    const uint32_t iv[4] = {iv0, iv1, iv2, iv3};
    return run_ctr(stream, nullptr, key, output, bytes, iv);
}

int secure_infer_gpu_auth_gate_do(hipStream_t stream, void* data, void* status, uint64_t bytes)
{
    if (!data || !status) return -1;
    return si::launch_auth_gate(stream, static_cast<uint8_t*>(data),
                                static_cast<const uint32_t*>(status), bytes) == hipSuccess ? 0 : -1;
}

int secure_infer_gpu_gcm_verify_xor_do(hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
                                       void* expected_tag, void* keystream, void* plaintext_output,
                                       void* status_output, uint64_t bytes, uint32_t iv0, uint32_t iv1,
                                       uint32_t iv2, uint32_t iv3)
{
    return secure_infer_gpu_gcm_verify_xor_aad_do(stream, ciphertext, key, hash_subkey, expected_tag, keystream,
                                                  plaintext_output, status_output, bytes, iv0, iv1, iv2, iv3,
                                                  nullptr, 0);
}

int secure_infer_gpu_gcm_verify_only_do(hipStream_t stream, void* ciphertext, void* key, void* hash_subkey,
                                        void* expected_tag, void* status_output, uint64_t bytes, uint32_t iv0,
                                        uint32_t iv1, uint32_t iv2, uint32_t iv3)
{
    return secure_infer_gpu_gcm_verify_only_aad_do(stream, ciphertext, key, hash_subkey, expected_tag,
                                                   status_output, bytes, iv0, iv1, iv2, iv3, nullptr, 0);
}

int secure_infer_gpu_gcm_verify_xor_batch_do(hipStream_t stream, void* key, void* hash_subkey,
                                             void* const* ciphertexts, void* const* expected_tags,
                                             void* const* keystreams, void* const* plaintext_outputs,
                                             void* const* status_outputs, void* const* aads, uint64_t bytes,
                                             uint64_t aad_bytes, const uint32_t* iv_words, uint32_t count)
{
    if (!key || !hash_subkey || !ciphertexts || !expected_tags || !keystreams || !plaintext_outputs ||
        !status_outputs || !iv_words || bytes == 0 || bytes > SI_MAX_RECORD_BYTES || (aad_bytes != 0 && !aads) ||
        count == 0 || count > SI_GCM_VERIFY_XOR_BATCH_MAX)
        return -1;
    for (uint32_t i = 0; i < count; ++i)
        if (!ciphertexts[i] || !expected_tags[i] || !keystreams[i] || !plaintext_outputs[i] || !status_outputs[i] ||
            (aad_bytes != 0 && !aads[i]))
            return -1;
    std::lock_guard<std::mutex> g(g_ctx_lock);
    DevCtx* c = ctx_for_device_key(stream, key, hash_subkey, npow_for(bytes, aad_bytes));
    if (!c) return -1;
    for (uint32_t i = 0; i < count; ++i)
        if (run_single_ctx(3, stream, c, ciphertexts[i], expected_tags[i], plaintext_outputs[i], status_outputs[i],
                           keystreams[i], bytes, iv_words + 4 * size_t(i), aad_bytes ? aads[i] : nullptr,
                           aad_bytes) != 0)
            return -1;
    return 0;
}

int secure_infer_gpu_keystream_batch_do(hipStream_t stream, void* key, void* const* outputs,
                                        const uint32_t* iv_words, uint64_t bytes, uint32_t count)
{
    if (!key || !outputs || !iv_words || bytes == 0 || count == 0 || count > SI_AES_KEYSTREAM_BATCH_MAX) return -1;
    for (uint32_t i = 0; i < count; ++i)
        if (!outputs[i]) return -1;
    std::lock_guard<std::mutex> g(g_ctx_lock);
    DevCtx* c = ctx_for_device_key(stream, key, nullptr, 1);
    if (!c) return -1;
    for (uint32_t i = 0; i < count; ++i)
        if (si::launch_ctr(stream, c->dev, nullptr, static_cast<uint8_t*>(outputs[i]), bytes,
                           iv_words + 4 * size_t(i)) != hipSuccess)
            return -1;
    return 0;
}

int secure_infer_gpu_ghash_do(hipStream_t stream, void* input, void* hash_subkey, void* output, void* aad,
                              void* tag_mask, void* expected_tag, void* keystream, void* plaintext_output,
                              void* status_output, uint64_t input_bytes, uint64_t aad_bytes, uint32_t flags)
{
    if (!input || !hash_subkey || !output || input_bytes == 0 || input_bytes > SI_MAX_RECORD_BYTES ||
        aad_bytes > SI_MAX_RECORD_BYTES || (aad_bytes != 0 && !aad) ||
        ((flags & SI_GHASH_FINALIZE_TAG) && !tag_mask) || ((flags & SI_GHASH_VERIFY_TAG) && !expected_tag) ||
        ((flags & SI_GHASH_XOR_ON_SUCCESS) && (!keystream || !plaintext_output)))
        return -1;
    std::lock_guard<std::mutex> g(g_ctx_lock);
    // The GHASH kernel reads the powers H^0 .. H^(T + 1) only.
    DevCtx* c = ctx_for_hash_subkey(stream, hash_subkey, SI_T + 2);
    if (!c) return -1;
    si::GhashJob j{};
    j.input = static_cast<const uint8_t*>(input);
    j.aad = static_cast<const uint8_t*>(aad);
    j.tag_mask = static_cast<const uint8_t*>(tag_mask);
    j.expected_tag = static_cast<const uint8_t*>(expected_tag);
    j.keystream = static_cast<const uint8_t*>(keystream);
    j.plaintext = static_cast<uint8_t*>(plaintext_output);
    j.status = static_cast<uint32_t*>(status_output);
    j.output = static_cast<uint8_t*>(output);
    j.input_bytes = input_bytes;
    j.aad_bytes = aad_bytes;
    j.flags = flags;
    return si::launch_ghash(stream, c->dev, j) == hipSuccess ? 0 : -1;
}

int secure_infer_gpu_key_agreement_do(hipStream_t stream, void* host_public, void* challenge, void* device_key,
                                      void* device_public, void* proof, void* status)
{
    if (!host_public || !challenge || !device_key || !device_public || !proof || !status) return -1;
    si::AgreeSeed seed{};
    if (RAND_bytes(seed.b, 32) != 1) return -1;
    // The entropy pool and its counter live on the stream's own schedule:
    // allocated, filled, hashed, zeroed and freed in stream order.
    const size_t pool_bytes = size_t(SI_AGREE_POOL_WORDS) * 4 + 16;
    uint32_t* pool = nullptr;
    if (hipMallocAsync(reinterpret_cast<void**>(&pool), pool_bytes, stream) != hipSuccess) {
        OPENSSL_cleanse(seed.b, sizeof(seed.b));
        return -1;
    }
    const hipError_t e = si::launch_agree(stream, static_cast<const uint8_t*>(host_public),
                                          static_cast<const uint8_t*>(challenge), seed, pool,
                                          pool + SI_AGREE_POOL_WORDS, static_cast<uint8_t*>(device_key),
                                          static_cast<uint8_t*>(device_public), static_cast<uint8_t*>(proof),
                                          static_cast<int32_t*>(status));
    OPENSSL_cleanse(seed.b, sizeof(seed.b));
    const hipError_t z = si::launch_zero_bytes(stream, reinterpret_cast<uint8_t*>(pool), uint32_t(pool_bytes));
    const hipError_t f = hipFreeAsync(pool, stream);
    return (e == hipSuccess && z == hipSuccess && f == hipSuccess) ? 0 : -1;
}

// ---------------------------------------------------------------- control plane

uint64_t secure_infer_new_transfer_ticket(void)
{
    const uint64_t t = g_next_ticket.fetch_add(1, std::memory_order_relaxed);
    if (t == 0) {
        fprintf(stderr, "[secure_infer] transfer ticket space exhausted\n");
        abort();
    }
    return t;
}

int secure_infer_derive_transfer_iv(const uint8_t base_iv[16], uint64_t session_nonce,
                                    uint64_t ticket, uint64_t block_offset, uint8_t out_iv[16])
{
    if (!base_iv || !out_iv || ticket == 0 || block_offset > UINT32_MAX - 2u) return -1;
    memcpy(out_iv, base_iv, 16);
    put_be64(out_iv + 4, session_nonce + ticket);
    put_be32(out_iv + 12, uint32_t(block_offset + 2));
    return 0;
}

void secure_infer_register_host_range_ex(const void* base, size_t bytes, uint32_t layer_id,
                                         uint32_t tensor_kind, size_t block_bytes)
{
    if (!base || bytes == 0) return;
    const uintptr_t b = reinterpret_cast<uintptr_t>(base);
    if (bytes > UINTPTR_MAX - b) return;
    std::lock_guard<std::mutex> g(g_ranges_lock);
    // Registering the same range again re-labels it (secure_infer.cpp:1066-1091).
    for (HostRange& r : g_ranges)
        if (r.begin == b && r.end == b + bytes) {
            r.layer = layer_id;
            r.kind = tensor_kind;
            r.block_bytes = block_bytes;
            return;
        }
    g_ranges.push_back(HostRange{b, b + bytes, layer_id, tensor_kind, block_bytes});
}

void secure_infer_register_host_range(const void* base, size_t bytes)
{
    secure_infer_register_host_range_ex(base, bytes, UINT32_MAX, UINT32_MAX, 0);
}

void secure_infer_clear_host_ranges(void)
{
    std::lock_guard<std::mutex> g(g_ranges_lock);
    g_ranges.clear();
}

int secure_infer_build_gcm_aad(const void* host_ptr, size_t bytes, uint8_t direction,
                               uint64_t transfer_ticket, uint64_t transfer_offset,
                               uint64_t session_nonce, uint8_t out[64])
{
    if (!out || !host_ptr || bytes == 0 || transfer_ticket == 0 || (direction != 1 && direction != 2))
        return 0;
    const uintptr_t begin = reinterpret_cast<uintptr_t>(host_ptr);
    uint32_t layer = UINT32_MAX, kind = UINT32_MAX;
    uint64_t block_id = begin, offset = 0;
    {
        std::lock_guard<std::mutex> g(g_ranges_lock);
        for (const HostRange& r : g_ranges) {
            if (begin < r.begin || begin + bytes > r.end) continue;
            const uint64_t rel = begin - r.begin;
            const uint64_t stride = r.block_bytes ? r.block_bytes : 1;
            layer = r.layer;
            kind = r.kind;
            block_id = rel / stride;
            offset = rel % stride;
            break;
        }
    }
    memset(out, 0, 64);
    out[0] = 'S'; out[1] = 'F'; out[2] = 'A'; out[3] = 'D';
    out[4] = 1;
    out[5] = direction;
    out[6] = uint8_t(kind & 0xff);
    put_be32(out + 8, layer);
    put_be64(out + 12, block_id);
    put_be64(out + 20, offset);
    put_be64(out + 28, bytes);
    put_be64(out + 36, transfer_ticket);
    put_be64(out + 44, transfer_offset);
    put_be64(out + 52, session_nonce);
    return 1;
}

int secure_infer_gcm_replay_reserve(uint64_t transfer_ticket)
{
    if (transfer_ticket == 0) return 1;
    if (replay_insert(transfer_ticket, transfer_ticket + 1)) return 1;
    fprintf(stderr, "[secure_infer] replayed transfer ticket rejected: %llu\n",
            static_cast<unsigned long long>(transfer_ticket));
    return 0;
}

// Groups nest per thread (secure_infer.cpp:5883-5903): the outermost begin
// announces the record count, the matching end issues the launch.
int secure_infer_h2d_layer_group_begin(size_t expected)
{
    if (t_group_depth++ == 0) t_group_expected = int64_t(expected);
    return 0;
}

int secure_infer_h2d_layer_group_end(void)
{
    if (t_group_depth == 0) return -1;
    if (--t_group_depth != 0) return 0;
    t_group_expected = -1;
    return si_internal::flush_pending_h2d() == 0 ? 0 : -1;
}

int secure_infer_recovery_track_layer(uint32_t layer, hipEvent_t event, const uint32_t* fail_count)
{
    if (!event || !fail_count) return -1;
    std::lock_guard<std::mutex> g(g_track_lock);
    g_tracked.emplace(layer, TrackedLayer{event, fail_count, false, g_job_id.load()});
    return 0;
}

int secure_infer_recovery_wait_layer_authentication(uint32_t layer)
{
    // Host-sealed records of the layer: statuses, one strict retry.
    bool found = false;
    const int rc_host = si_internal::wait_observed_layer(layer, &found);
    // Device-resident records of the layer: a fail count (no host copy to
    // retry from).
    std::vector<TrackedLayer> recs;
    {
        std::lock_guard<std::mutex> g(g_track_lock);
        auto range = g_tracked.equal_range(layer);
        for (auto it = range.first; it != range.second; ++it) recs.push_back(it->second);
        g_tracked.erase(range.first, range.second);
    }
    int rc = 0;
    for (const TrackedLayer& t : recs) {
        uint32_t fails = 1;
        if (hipEventSynchronize(t.event) != hipSuccess ||
            hipMemcpy(&fails, t.fail_count, 4, hipMemcpyDeviceToHost) != hipSuccess)
            rc = -1;
        else if (fails != 0)
            rc = -1;
        if (t.owned) (void)hipEventDestroy(t.event);
    }
    return (rc != 0 || rc_host != 0) ? -1 : 0;
}

void secure_infer_recovery_set_job_id(uint64_t job_id) { g_job_id.store(job_id); }

int secure_infer_recovery_wait_job_authentication(uint64_t job_id)
{
    // Every record of the job, on every layer, without retries
    // (secure_infer.cpp:7336-7372): 1 if all authenticated, 0 if any failed,
    // -1 if the job has no observed records.
    std::vector<TrackedLayer> recs;
    {
        std::lock_guard<std::mutex> g(g_track_lock);
        for (auto it = g_tracked.begin(); it != g_tracked.end();) {
            if (it->second.job_id == job_id) {
                recs.push_back(it->second);
                it = g_tracked.erase(it);
            } else {
                ++it;
            }
        }
    }
    bool valid = true;
    for (const TrackedLayer& t : recs) {
        uint32_t fails = 1;
        if (hipEventSynchronize(t.event) != hipSuccess ||
            hipMemcpy(&fails, t.fail_count, 4, hipMemcpyDeviceToHost) != hipSuccess || fails != 0)
            valid = false;
        if (t.owned) (void)hipEventDestroy(t.event);
    }
    bool found = !recs.empty();
    const int host = si_internal::wait_observed_job(job_id, &found);
    if (!found) return -1;
    return (valid && host == 1) ? 1 : 0;
}

int secure_infer_gpu_set_chunk_rows(int jmax)
{
    if (jmax < 1 || jmax > 256) return -1;
    g_min_rows.store(jmax, std::memory_order_relaxed);
    return 0;
}

int secure_infer_gpu_set_straddle_rows(int rows)
{
    if (rows < 0 || rows > 256) return -1;
    g_straddle_rows.store(uint32_t(rows), std::memory_order_relaxed);
    return 0;
}

int secure_infer_gpu_layout(uint32_t nrec, uint64_t bytes, uint64_t aad_bytes, uint32_t cus, uint32_t* info_out,
                            uint32_t* starts_out, uint32_t cap)
{
    if (!info_out || nrec == 0 || bytes == 0 || bytes > SI_MAX_RECORD_BYTES || aad_bytes > SI_MAX_RECORD_BYTES || cus == 0 ||
        cus > SI_MAX_WG)
        return -1;
    const si::Sched s = make_sched_uncached(nrec, bytes, aad_bytes, cus, g_min_rows.load(std::memory_order_relaxed),
                                            g_straddle_rows.load(std::memory_order_relaxed));
    info_out[0] = s.nwg;
    info_out[1] = s.rows;
    info_out[2] = s.use_starts;
    info_out[3] = s.pairs;
    info_out[4] = s.ek_row0;
    if (s.use_starts) {
        if (!starts_out || cap < s.nwg + 1) return -1;
        memcpy(starts_out, s.starts, (size_t(s.nwg) + 1) * sizeof(uint32_t));
    }
    return 0;
}

}  // extern "C"

namespace si_internal {

void session_hold(si_session* s) { s->holds.fetch_add(1, std::memory_order_acq_rel); }

void session_release(si_session* s) { s->holds.fetch_sub(1, std::memory_order_acq_rel); }

uint32_t session_holds(const si_session* s) { return s->holds.load(std::memory_order_acquire); }

SessionKeys session_keys(const si_session* s)
{
    SessionKeys k{};
    memcpy(k.key, s->ctx->key, 16);
    put_be32(k.salt, s->salt_word);
    k.nonce = s->session_nonce;
    k.max_record_bytes = s->max_record_bytes;
    return k;
}

uint64_t reserve_tickets(uint32_t n)
{
    const uint64_t t = g_next_ticket.fetch_add(n, std::memory_order_relaxed);
    if (t == 0 || t + n < t) {
        fprintf(stderr, "[secure_infer] transfer ticket space exhausted\n");
        abort();
    }
    return t;
}

bool replay_reserve_range(uint64_t t0, uint64_t n) { return replay_insert(t0, t0 + n); }

bool group_open() { return t_group_depth > 0; }

int64_t group_expected() { return t_group_expected; }

uint64_t current_job_id() { return g_job_id.load(); }

}  // namespace si_internal
