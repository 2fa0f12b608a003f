// tier_driver.cpp -- the HBM expert tier driven the way the engine's store drives it, from
// two threads, checked against the CPU oracle.  Built against the library (plain, or its
// host side under AddressSanitizer / ThreadSanitizer: tests/native/Makefile).
//
// A RAM tier of pinned slots stands in for ExpertStore (src/store/expert_store.cpp):
// lookup() fills a free or least-recently-used slot with the expert's blob (generated
// from (layer, eid), as a pread would bring it), calling mvllm_hip_host_reuse before it
// rewrites a slot and queueing the evicted expert as a REPIN event; prefetch() loads the
// next layer's experts and hands them to mvllm_hip_prefetch (the store's
// prefetch_one_async path).  Slots are pinned by leases while a call or a prefetch reads
// them, and a slot being loaded is handed to no one until its load ends (the store's
// loading state).
//
//   store thread:   for each layer l + 1 ahead of the compute thread: prefetch its
//                   experts; drain REPIN events into mvllm_hip_repin.
//   compute thread: for each layer l: lease its experts (lookup), run the drop-in
//                   mvllm_hip_moe_block on their host pointers (resident blobs are read
//                   from HBM, the rest copied in), release; every few layers also the
//                   device-resident form (mvllm_hip_tier_table +
//                   mvllm_hip_moe_block_routed_dev on segments in device memory); check
//                   outputs against orc_moe_block.
//
// Exit status 0 when every checked output is within the bar, 1 otherwise.
#include "../../include/mvllm_hip.h"
#include "../../oracle/moe_oracle.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include <unistd.h>

namespace {

constexpr int kFmt = 7, kD = 512, kI = 256, kExperts = 24, kLayers = 6, kTopk = 4, kTok = 5;
constexpr int kSlotsPerLayer = 20;  // a call's experts fit; fewer than the layer's 24

long long g_blob = 0;
long long g_off[6];

uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// The blob of (layer, eid): random codes, ue8m0 scales in [118, 124].
void fill_blob(uint8_t *p, int layer, int eid) {
    uint32_t s = mix32((uint32_t)(layer * 1000003 + eid * 7919 + 17));
    for (long long i = 0; i < g_blob; ++i) {
        s = mix32(s + (uint32_t)i);
        p[i] = (uint8_t)s;
    }
    // scale pieces: gate_s, up_s, down_s (geometry offsets 1, 3, 5); each piece ends where
    // the next piece of the blob layout begins
    for (int k : {1, 3, 5}) {
        long long end = g_blob;
        for (long long o : g_off)
            if (o > g_off[k])
                end = std::min(end, o);
        for (long long i = g_off[k]; i < end; ++i)
            p[i] = (uint8_t)(118 + p[i] % 7);
    }
}

struct RamTier {
    struct Slot {
        uint8_t *base = nullptr;
        int eid = -1, pins = 0;
        bool loading = false;
        unsigned long long used = 0;
    };
    std::mutex mu;
    std::condition_variable loaded;
    std::vector<std::vector<Slot>> layers;
    std::deque<std::pair<int, int>> repin;
    unsigned long long clock = 1;
    std::atomic<int> reuse_calls{0};

    bool open() {
        layers.assign(kLayers, std::vector<Slot>(kSlotsPerLayer));
        for (auto &L : layers)
            for (auto &s : L) {
                s.base = static_cast<uint8_t *>(mvllm_hip_host_alloc((size_t)g_blob));
                if (!s.base)
                    return false;
            }
        return true;
    }
    void close() {
        for (auto &L : layers)
            for (auto &s : L)
                mvllm_hip_host_free(s.base);
    }
    // the slot holding (layer, eid), loading it when absent; leased when pin (release()
    // ends the lease).  A slot that another thread is loading is waited for.
    uint8_t *lookup(int layer, int eid, bool pin) {
        std::unique_lock<std::mutex> lk(mu);
        auto &L = layers[layer];
        for (;;) {
            Slot *hit = nullptr;
            for (auto &s : L)
                if (s.eid == eid)
                    hit = &s;
            if (!hit)
                break;
            if (hit->loading) {
                loaded.wait(lk);
                continue;  // the slot may have changed hands meanwhile
            }
            hit->used = clock++;
            hit->pins += pin;
            return hit->base;
        }
        Slot *v = nullptr;
        for (auto &s : L)
            if (s.pins == 0 && !s.loading && (!v || s.used < v->used))
                v = &s;
        if (!v)
            return nullptr;  // every slot leased
        const int old = v->eid;
        v->eid = eid;
        v->used = clock++;
        v->loading = true;
        v->pins += 1;  // held during the load
        lk.unlock();
        // the slot is about to be rewritten: copies from its old contents must finish
        if (mvllm_hip_host_reuse(v->base, (size_t)g_blob) < 0)
            std::fprintf(stderr, "host_reuse: %s\n", mvllm_hip_last_error());
        reuse_calls++;
        fill_blob(v->base, layer, eid);
        lk.lock();
        v->loading = false;
        v->pins -= 1;
        v->pins += pin;
        if (old >= 0)
            repin.emplace_back(layer, old);
        loaded.notify_all();
        return v->base;
    }
    void release(uint8_t *base) {
        std::lock_guard<std::mutex> lk(mu);
        for (auto &L : layers)
            for (auto &s : L)
                if (s.base == base && s.pins > 0) {
                    s.pins -= 1;
                    return;
                }
    }
    std::vector<int> take_repin() {
        std::lock_guard<std::mutex> lk(mu);
        std::vector<int> out;
        for (auto &e : repin) {
            out.push_back(e.first);
            out.push_back(e.second);
        }
        repin.clear();
        return out;
    }
};

// the experts and routing of (step, layer): kTok tokens, top-k distinct experts each
struct Route {
    std::vector<int> idx;
    std::vector<float> wt;
};

Route route_of(int step, int layer) {
    Route r;
    r.idx.resize(kTok * kTopk);
    r.wt.resize(kTok * kTopk);
    for (int t = 0; t < kTok; ++t) {
        uint32_t s = mix32((uint32_t)(step * 7777 + layer * 131 + t));
        int k = 0;
        while (k < kTopk) {
            s = mix32(s + 1);
            const int e = (int)(s % kExperts);
            bool dup = false;
            for (int j = 0; j < k; ++j)
                dup |= r.idx[t * kTopk + j] == e;
            if (dup)
                continue;
            r.idx[t * kTopk + k] = e;
            r.wt[t * kTopk + k] = 0.1f + 0.2f * (float)(s % 5);
            ++k;
        }
    }
    return r;
}

float rel_err(const std::vector<float> &a, const std::vector<float> &b) {
    double m = 0, r = 0;
    for (size_t i = 0; i < a.size(); ++i) {
        m = std::max(m, (double)std::fabs(a[i] - b[i]));
        r = std::max(r, (double)std::fabs(b[i]));
    }
    return (float)(r > 0 ? m / r : m);
}

// The segments of a route on the host (mvllm_moe_segments), the oracle's output for them
// from the blobs (regenerated, independent of the tiers), and the x rows.
struct Call {
    int nb = 0, n_rows = 0;
    std::vector<int> eids, xoff, nr, rows;
    std::vector<float> rw, x, xg, exp;
};

Call make_call(int step, int layer) {
    Call c;
    Route r = route_of(step, layer);
    c.eids.resize(kExperts);
    c.xoff.resize(kExperts);
    c.nr.resize(kExperts);
    c.rows.resize(kTok * kTopk);
    c.rw.resize(kTok * kTopk);
    c.nb = mvllm_moe_segments(r.idx.data(), r.wt.data(), kTok, kTopk, c.eids.data(),
                              c.xoff.data(), c.nr.data(), c.rows.data(), c.rw.data(), kExperts,
                              kTok * kTopk, &c.n_rows);
    c.x.resize((size_t)kTok * kD);
    for (size_t i = 0; i < c.x.size(); ++i)
        c.x[i] = (float)((int)(mix32((uint32_t)(step * 31 + layer * 7 + i)) % 2001) - 1000) / 500.f;
    c.xg.resize((size_t)c.n_rows * kD);
    for (int j = 0; j < c.n_rows; ++j)
        std::memcpy(&c.xg[(size_t)j * kD], &c.x[(size_t)c.rows[j] * kD], kD * sizeof(float));
    std::vector<std::vector<uint8_t>> blobs(c.nb, std::vector<uint8_t>((size_t)g_blob));
    std::vector<const void *> g(c.nb), u(c.nb), d(c.nb);
    std::vector<const float *> gs(c.nb), us(c.nb), ds(c.nb);
    for (int i = 0; i < c.nb; ++i) {
        fill_blob(blobs[i].data(), layer, c.eids[i]);
        const uint8_t *b = blobs[i].data();
        g[i] = b + g_off[0];
        gs[i] = reinterpret_cast<const float *>(b + g_off[1]);
        u[i] = b + g_off[2];
        us[i] = reinterpret_cast<const float *>(b + g_off[3]);
        d[i] = b + g_off[4];
        ds[i] = reinterpret_cast<const float *>(b + g_off[5]);
    }
    c.exp.assign((size_t)kTok * kD, 0.f);
    orc_moe_block(c.nb, kD, kI, kFmt, 32, g.data(), u.data(), d.data(), gs.data(), us.data(),
                  ds.data(), c.xg.data(), c.xoff.data(), c.nr.data(), c.rows.data(), c.rw.data(),
                  c.exp.data(), kTok, ORC_ACT_SITU, 4.f, 25.f);
    return c;
}

// ---- host-only checks (no device): the container reader on mutated headers and the
// segment builders against the oracle ------------------------------------------------

void put_le64(std::string &o, uint64_t v) {
    for (int i = 0; i < 8; ++i)
        o += (char)((v >> (8 * i)) & 0xff);
}

// A K3 container of one expert (layer 0) with D = I = 32, as the reference's tests write
// one (tests/test_host.cpp:3636-3668).
std::string k3_container(std::string *header_out) {
    static const char *mats[3] = {"w1", "w2", "w3"};
    static const char *half[2] = {"packed", "scale"};
    const long long want[6] = {32 * 16, 32, 32 * 16, 32, 32 * 16, 32};
    std::string h = "{\"__metadata__\":{\"format\":\"pt\"}";
    long long off = 0;
    for (int k = 0; k < 6; ++k) {
        h += ",\"model.layers.0.block_sparse_moe.experts.0.";
        h += mats[k / 2];
        h += ".weight_";
        h += half[k & 1];
        h += "\":{\"dtype\":\"U8\",\"shape\":[" + std::to_string(want[k]) +
             "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + want[k]) +
             "]}";
        off += want[k];
    }
    h += "}";
    if (header_out)
        *header_out = h;
    std::string f;
    put_le64(f, h.size());
    f += h;
    for (long long i = 0; i < off; ++i)
        f += (char)(i * 7);
    return f;
}

int host_checks(int iters, uint32_t seed) {
    char dir[] = "/tmp/mvllm_st_XXXXXX";
    if (!mkdtemp(dir))
        return 2;
    const std::string path = std::string(dir) + "/m.safetensors";
    std::string header;
    const std::string good = k3_container(&header);
    auto write = [&](const std::string &bytes) {
        FILE *f = std::fopen(path.c_str(), "wb");
        std::fwrite(bytes.data(), 1, bytes.size(), f);
        std::fclose(f);
    };
    int failures = 0;
    int file[6];
    long long off[6], by[6];
    char err[512];
    write(good);
    if (mvllm_st_expert_pieces(dir, "", 7, 32, 32, 0, 1, 1, file, off, by, nullptr, 0, err,
                               sizeof(err)) != 1) {
        std::fprintf(stderr, "good container refused: %s\n", err);
        ++failures;
    }
    // offsets of 19 and 20 digits past the 64-bit range: an error, not an exception
    for (const char *big : {"9999999999999999999", "18446744073709551616",
                            "-9223372036854775809"}) {
        std::string h = header;
        const size_t at = h.find("\"data_offsets\":[0,");
        const size_t e = h.find(']', at);
        h.replace(at, e - at, std::string("\"data_offsets\":[0,") + big);
        std::string b;
        put_le64(b, h.size());
        b += h;
        b += good.substr(8 + header.size());
        write(b);
        err[0] = '\0';
        if (mvllm_st_expert_pieces(dir, "", 7, 32, 32, 0, 1, 1, file, off, by, nullptr, 0, err,
                                   sizeof(err)) != -1 ||
            !std::strstr(err, "out of range")) {
            std::fprintf(stderr, "offset %s: not refused as out of range (%s)\n", big, err);
            ++failures;
        }
    }
    // mutated containers: byte flips in the header, truncations, bad lengths; each must
    // give an answer (pieces or an error), never a crash
    uint32_t s = 12345 + seed;
    int accepted = 0;
    for (int it = 0; it < iters; ++it) {
        std::string b = good;
        s = mix32(s + (uint32_t)it);
        const int kind = (int)(s % 4);
        if (kind == 0) {  // flip bytes inside the header
            for (int j = 0; j < 1 + (int)(s >> 8) % 4; ++j) {
                s = mix32(s);
                b[8 + s % header.size()] = (char)(s >> 16);
            }
        } else if (kind == 1) {  // truncate anywhere
            b.resize(s % good.size());
        } else if (kind == 2) {  // another header length
            const uint64_t n = (s >> 4) % (header.size() * 2 + 16);
            for (int i = 0; i < 8; ++i)
                b[i] = (char)((n >> (8 * i)) & 0xff);
        } else {  // drop a span of the header
            const size_t a = 8 + s % header.size(), n = 1 + (s >> 12) % 16;
            b.erase(a, std::min(n, b.size() - a));
        }
        write(b);
        accepted += mvllm_st_expert_pieces(dir, "", 7, 32, 32, 0, 1, 1, file, off, by, nullptr, 0,
                                           err, sizeof(err)) == 1;
    }
    std::remove(path.c_str());
    rmdir(dir);
    // segments: the library's host builder against the oracle's on random routes
    for (int it = 0; it < iters; ++it) {
        const int T = 1 + it % 37, k = 1 + it % 8, E = 4 + it % 61;
        std::vector<int> idx(T * k);
        std::vector<float> wt(T * k);
        for (int i = 0; i < T * k; ++i) {
            s = mix32(s + 1);
            idx[i] = (int)(s % (E + 2)) - 1;  // -1 ids and repeats included
            wt[i] = (float)((int)(s >> 8) % 7 - 2) * 0.25f;  // zero and cancelling sums
        }
        std::vector<int> e1(E + 2), x1(E + 2), n1(E + 2), r1(T * k), e2(E + 2), x2(E + 2),
            n2(E + 2), r2(T * k);
        std::vector<float> w1(T * k), w2(T * k);
        int m1 = 0, m2 = 0;
        const int a = mvllm_moe_segments(idx.data(), wt.data(), T, k, e1.data(), x1.data(),
                                         n1.data(), r1.data(), w1.data(), E + 2, T * k, &m1);
        const int b = orc_moe_segments(idx.data(), wt.data(), T, k, e2.data(), x2.data(),
                                       n2.data(), r2.data(), w2.data(), E + 2, T * k, &m2);
        bool same = a == b && m1 == m2;
        for (int i = 0; same && i < a; ++i)
            same = e1[i] == e2[i] && x1[i] == x2[i] && n1[i] == n2[i];
        for (int j = 0; same && j < m1; ++j)
            same = r1[j] == r2[j] && std::memcmp(&w1[j], &w2[j], 4) == 0;
        if (!same) {
            std::fprintf(stderr, "segments differ from the oracle (T %d k %d E %d)\n", T, k, E);
            ++failures;
        }
    }
    std::printf("host checks: %d mutated containers (%d accepted), %d segment cases, %d "
                "failures\n", iters, accepted, iters, failures);
    return failures ? 1 : 0;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc > 1 && std::strcmp(argv[1], "host") == 0)
        return host_checks(argc > 2 ? std::atoi(argv[2]) : 2000, 0);
    if (argc > 1 && std::strcmp(argv[1], "host-threads") == 0) {
        // the host-only entry points from several threads at once, with option changes,
        // counter reads and refused device calls (no device: their argument checks and
        // error text) in between
        const int iters = argc > 2 ? std::atoi(argv[2]) : 500;
        std::atomic<int> bad{0};
        std::vector<std::thread> th;
        for (int t = 0; t < 4; ++t)
            th.emplace_back([&, t] { bad += host_checks(iters, 1000u * (uint32_t)(t + 1)); });
        th.emplace_back([&] {
            double sv[19];
            for (int i = 0; i < iters; ++i) {
                mvllm_hip_set_option("combine_ordered", i & 1);
                mvllm_hip_set_option("mode", i % 3);
                mvllm_hip_stats(sv, 19);
                if (i % 7 == 0)
                    mvllm_hip_stats_reset();
                // refused without a device; the error text is per thread
                if (mvllm_hip_promote(nullptr, 0, 0, 0) != 0 ||
                    std::strstr(mvllm_hip_last_error(), "promote") == nullptr)
                    bad++;
                if (mvllm_hip_slab_free(1000 + i) != 0)
                    bad++;
            }
        });
        for (auto &t : th)
            t.join();
        mvllm_hip_set_option("combine_ordered", 0);
        mvllm_hip_set_option("mode", 0);
        std::printf("host threads: %d failures\n", bad.load());
        return bad.load() ? 1 : 0;
    }
    const int steps = argc > 1 ? std::atoi(argv[1]) : 3;
    if (!mvllm_hip_init(0)) {
        std::fprintf(stderr, "init: %s\n", mvllm_hip_last_error());
        return 2;
    }
    g_blob = mvllm_expert_geom(kFmt, kD, kI, g_off);
    // HBM budget for about two layers' worth of a call's experts: promotions evict
    const size_t budget = (size_t)g_blob * 2 * kSlotsPerLayer;
    mvllm_hip_set_expert_budget(budget);
    RamTier ram;
    if (!ram.open()) {
        std::fprintf(stderr, "host_alloc failed\n");
        return 2;
    }
    std::atomic<int> layer_done{-1}, failures{0}, checked{0};
    std::mutex mu;
    std::condition_variable cv;
    const int total = steps * kLayers;

    std::thread store([&] {
        for (int n = 1; n < total; ++n) {
            {
                std::unique_lock<std::mutex> lk(mu);
                // layer n - 1 is computing (n - 2 done): prefetch layer n meanwhile
                cv.wait(lk, [&] { return layer_done.load() >= n - 2; });
            }
            const int step = n / kLayers, layer = n % kLayers;
            Call c = make_call(step, layer);
            std::vector<int> ls, es;
            std::vector<const void *> hb;
            std::vector<size_t> by;
            // leased until the promotions are enqueued: the compute thread may not
            // rewrite a slot between its load and the copy out of it
            for (int i = 0; i < c.nb; ++i) {
                uint8_t *p = ram.lookup(layer, c.eids[i], true);
                if (!p)
                    continue;
                ls.push_back(layer);
                es.push_back(c.eids[i]);
                hb.push_back(p);
                by.push_back((size_t)g_blob);
            }
            if (mvllm_hip_prefetch((int)es.size(), ls.data(), es.data(), hb.data(), by.data()) <
                0) {
                std::fprintf(stderr, "prefetch: %s\n", mvllm_hip_last_error());
                failures++;
            }
            for (const void *p : hb)
                ram.release(static_cast<uint8_t *>(const_cast<void *>(p)));
            std::vector<int> rp = ram.take_repin();
            if (mvllm_hip_repin((int)rp.size() / 2, rp.data()) < 0)
                failures++;
        }
    });

    void *table = nullptr, *dsegs = nullptr;
    float *dx = nullptr, *dout = nullptr;
    hipStream_t st = nullptr;
    bool dev_ok = hipMalloc(&table, kExperts * sizeof(void *)) == hipSuccess &&
                  hipMalloc(&dsegs, 64 * 1024) == hipSuccess &&
                  hipMalloc(&dx, (size_t)kTok * kD * 4) == hipSuccess &&
                  hipMalloc(&dout, (size_t)kTok * kD * 4) == hipSuccess &&
                  hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess;
    if (!dev_ok) {
        std::fprintf(stderr, "device allocation failed\n");
        return 2;
    }
    for (int n = 0; n < total; ++n) {
        const int step = n / kLayers, layer = n % kLayers;
        Call c = make_call(step, layer);
        // lease the layer's experts, then the drop-in host entry on their host pointers
        std::vector<uint8_t *> lease(c.nb);
        std::vector<const void *> g(c.nb), u(c.nb), d(c.nb);
        std::vector<const float *> gs(c.nb), us(c.nb), ds(c.nb);
        for (int i = 0; i < c.nb; ++i) {
            lease[i] = ram.lookup(layer, c.eids[i], true);
            // the store's leases are short (until its promotions are enqueued)
            for (int tries = 0; !lease[i] && tries < 20000; ++tries) {
                usleep(100);
                lease[i] = ram.lookup(layer, c.eids[i], true);
            }
            if (!lease[i]) {
                std::fprintf(stderr, "all slots leased\n");
                return 2;
            }
            const uint8_t *b = lease[i];
            g[i] = b + g_off[0];
            gs[i] = reinterpret_cast<const float *>(b + g_off[1]);
            u[i] = b + g_off[2];
            us[i] = reinterpret_cast<const float *>(b + g_off[3]);
            d[i] = b + g_off[4];
            ds[i] = reinterpret_cast<const float *>(b + g_off[5]);
        }
        std::vector<float> out((size_t)kTok * kD, 0.f);
        if (!mvllm_hip_moe_block(c.nb, kD, kI, kFmt, 32, g.data(), u.data(), d.data(), gs.data(),
                                 us.data(), ds.data(), c.xg.data(), c.xoff.data(), c.nr.data(),
                                 c.rows.data(), c.rw.data(), out.data(), kTok, 2, 4.f, 25.f)) {
            std::fprintf(stderr, "moe_block: %s\n", mvllm_hip_last_error());
            failures++;
        }
        for (uint8_t *p : lease)
            ram.release(p);
        const float e1 = rel_err(out, c.exp);
        checked++;
        if (!(e1 < 2e-5f)) {
            std::fprintf(stderr, "step %d layer %d: host entry rel_err %g\n", step, layer, e1);
            failures++;
        }
        // every other layer: the device-resident form from the HBM tier's table (experts
        // not resident in HBM are skipped, so compare only when all are)
        if (n % 2 == 0) {
            int nres = 0;
            if (!mvllm_hip_tier_table(layer, kExperts, static_cast<void **>(table), &nres, st)) {
                std::fprintf(stderr, "tier_table: %s\n", mvllm_hip_last_error());
                failures++;
            }
            // segments into device memory: counts, eids, xoff, nr, rows, rw
            char *s = static_cast<char *>(dsegs);
            int counts[2] = {c.nb, c.n_rows};
            (void)hipMemcpyAsync(s, counts, 8, hipMemcpyHostToDevice, st);
            (void)hipMemcpyAsync(s + 256, c.eids.data(), kExperts * 4, hipMemcpyHostToDevice, st);
            (void)hipMemcpyAsync(s + 512, c.xoff.data(), kExperts * 4, hipMemcpyHostToDevice, st);
            (void)hipMemcpyAsync(s + 768, c.nr.data(), kExperts * 4, hipMemcpyHostToDevice, st);
            (void)hipMemcpyAsync(s + 1024, c.rows.data(), kTok * kTopk * 4, hipMemcpyHostToDevice, st);
            (void)hipMemcpyAsync(s + 2048, c.rw.data(), kTok * kTopk * 4, hipMemcpyHostToDevice, st);
            (void)hipMemcpyAsync(dx, c.x.data(), (size_t)kTok * kD * 4, hipMemcpyHostToDevice, st);
            (void)hipMemsetAsync(dout, 0, (size_t)kTok * kD * 4, st);
            const int ok = mvllm_hip_moe_block_routed_dev(
                kD, kI, kFmt, static_cast<const void *const *>(table), kExperts,
                reinterpret_cast<int *>(s), reinterpret_cast<int *>(s + 256),
                reinterpret_cast<int *>(s + 512), reinterpret_cast<int *>(s + 768), kExperts,
                reinterpret_cast<int *>(s + 1024), reinterpret_cast<float *>(s + 2048),
                kTok * kTopk, dx, dout, kTok, 2, 4.f, 25.f, nullptr, st);
            {
                // the table is still open here while the store thread promotes: the tier's
                // device memory (resident plus parked blocks) stays within the budget
                double sv[19];
                if (mvllm_hip_stats(sv, 19) == 19 && sv[17] > (double)budget) {
                    std::fprintf(stderr, "step %d layer %d: tier holds %.0f bytes, budget %zu\n",
                                 step, layer, sv[17], budget);
                    failures++;
                }
            }
            mvllm_hip_tier_table_done(layer, st);
            std::vector<float> out2((size_t)kTok * kD);
            std::vector<void *> seen(kExperts);
            (void)hipMemcpyAsync(out2.data(), dout, out2.size() * 4, hipMemcpyDeviceToHost, st);
            (void)hipMemcpyAsync(seen.data(), table, kExperts * sizeof(void *),
                                 hipMemcpyDeviceToHost, st);
            (void)hipStreamSynchronize(st);
            // the call's experts all in the table the routed call read (the store thread
            // promotes and evicts meanwhile, so residency is read from that table itself)
            int all = 1;
            for (int i = 0; i < c.nb; ++i)
                all &= seen[c.eids[i]] != nullptr;
            if (!ok) {
                std::fprintf(stderr, "routed: %s\n", mvllm_hip_last_error());
                failures++;
            } else if (all) {
                const float e2 = rel_err(out2, c.exp);
                checked++;
                if (!(e2 < 2e-5f)) {
                    std::fprintf(stderr, "step %d layer %d: routed rel_err %g (resident %d)\n",
                                 step, layer, e2, nres);
                    failures++;
                }
            }
        }
        {
            std::lock_guard<std::mutex> lk(mu);
            layer_done = n;
        }
        cv.notify_all();
    }
    store.join();
    double sv[17];
    mvllm_hip_stats(sv, 17);
    std::printf("tier_driver: %d layer calls, %d outputs checked, %d failures; promotions %.0f, "
                "resident hits %.0f, misses %.0f, evictions %.0f, slot reuses %d\n",
                total, checked.load(), failures.load(), sv[5], sv[6], sv[7], sv[8],
                ram.reuse_calls.load());
    (void)hipStreamDestroy(st);
    (void)hipFree(table);
    (void)hipFree(dsegs);
    (void)hipFree(dx);
    (void)hipFree(dout);
    ram.close();
    mvllm_hip_shutdown();
    return failures.load() == 0 ? 0 : 1;
}
