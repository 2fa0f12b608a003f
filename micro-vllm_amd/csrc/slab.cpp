// slab.cpp -- routed experts from safetensors containers into one device slab.
//
// The reference registers each expert's six pieces (file, offset, bytes) with its
// ExpertStore, which reads them into pinned host slots on demand
// (src/model/glm53.cpp:1829-1871, src/model/kimi_k3.cpp:1881-1934,
// src/store/expert_store.cpp).  Here a layer range of experts goes to HBM at once: one
// device allocation of n_blobs blobs, each the six pieces back to back in the reference's
// blob layout (so one blob address and the blob geometry give all six pointers), plus a
// device table of blob addresses indexed (layer - layer0) * n_experts + expert.  The
// pieces are read with pread into two pinned staging buffers while the previous buffer
// is copied to the device: file reads overlap the host-to-device copies.
#include "../../include/mvllm_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include <fcntl.h>
#include <unistd.h>

#include "st_index.hpp"

namespace mvllm_hip {
void set_error(const std::string &s);  // mvllm_hip.cpp: the text of mvllm_hip_last_error

namespace {

struct Slab {
    int fmt = 0, D = 0, I = 0, layer0 = 0, layer1 = 0, n_experts = 0;
    long long blob_bytes = 0, stride = 0;
    void *base = nullptr;
    void *table = nullptr;  // device: const void *[n_blobs]
};

std::mutex g_mu;
std::map<long long, Slab> g_slabs;
long long g_next = 1;

constexpr size_t kStage = size_t(32) << 20;  // bytes per pinned staging buffer

// A contiguous span of one file that lands contiguously in the slab.
struct Span {
    int file;
    uint64_t off, bytes;
    size_t dst;  // byte offset in the slab
};

bool read_all(int fd, char *dst, size_t n, off_t off) {
    while (n) {
        const ssize_t r = ::pread(fd, dst, n, off);
        if (r < 0 && errno == EINTR)
            continue;
        if (r <= 0)
            return false;
        dst += r;
        n -= (size_t)r;
        off += r;
    }
    return true;
}

// Streams the spans into the device slab; 1 ok, 0 with the error set.
int stream_spans(const std::vector<StFileIdx> &files, const std::vector<Span> &spans, char *dev) {
    std::vector<int> fds(files.size(), -1);
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t st = nullptr;
    bool used[2] = {false, false};
    std::string err;
    auto fail = [&](const std::string &s) {
        if (err.empty())
            err = s;
        return false;
    };
    auto hip_ok = [&](hipError_t e, const char *what) {
        return e == hipSuccess || fail(std::string(what) + ": " + hipGetErrorString(e));
    };
    bool ok = hip_ok(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    for (int b = 0; ok && b < 2; ++b)
        ok = hip_ok(hipHostMalloc(&stage[b], kStage, hipHostMallocDefault), "hipHostMalloc") &&
             hip_ok(hipEventCreateWithFlags(&done[b], hipEventDisableTiming), "hipEventCreate");
    int buf = 0;
    for (size_t s = 0; ok && s < spans.size(); ++s) {
        const Span &sp = spans[s];
        if (fds[sp.file] < 0) {
            fds[sp.file] = ::open(files[sp.file].path.c_str(), O_RDONLY | O_CLOEXEC);
            if (fds[sp.file] < 0) {
                ok = fail("open(" + files[sp.file].path + "): " + std::strerror(errno));
                break;
            }
        }
        for (uint64_t at = 0; ok && at < sp.bytes; at += kStage) {
            const size_t n = (size_t)std::min<uint64_t>(kStage, sp.bytes - at);
            if (used[buf])  // the copy that last read this buffer has finished
                ok = hip_ok(hipEventSynchronize(done[buf]), "hipEventSynchronize");
            if (!ok)
                break;
            if (!read_all(fds[sp.file], static_cast<char *>(stage[buf]), n,
                          (off_t)(sp.off + at))) {
                ok = fail("read(" + files[sp.file].path + "): short read");
                break;
            }
            ok = hip_ok(hipMemcpyAsync(dev + sp.dst + at, stage[buf], n, hipMemcpyHostToDevice,
                                       st),
                        "hipMemcpyAsync") &&
                 hip_ok(hipEventRecord(done[buf], st), "hipEventRecord");
            used[buf] = true;
            buf ^= 1;
        }
    }
    if (st)
        ok = hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize") && ok;
    for (int b = 0; b < 2; ++b) {
        if (stage[b])
            (void)hipHostFree(stage[b]);
        if (done[b])
            (void)hipEventDestroy(done[b]);
    }
    if (st)
        (void)hipStreamDestroy(st);
    for (int fd : fds)
        if (fd >= 0)
            ::close(fd);
    if (!ok)
        set_error("slab_load: " + err);
    return ok ? 1 : 0;
}

}  // namespace
}  // namespace mvllm_hip

using namespace mvllm_hip;

static long long slab_load_impl(const char *dir, const char *prefix, int fmt, int D, int I,
                                int layer0, int layer1, int n_experts) {
    set_error("");
    if (!mvllm_hip_available()) {
        set_error("slab_load: mvllm_hip_init not called");
        return 0;
    }
    if (!dir || (fmt != 4 && fmt != 7) || D < 1 || I < 1 || layer1 <= layer0 || layer0 < 0 ||
        n_experts < 1) {
        set_error("slab_load: bad arguments");
        return 0;
    }
    std::string err;
    std::vector<StFileIdx> files;
    std::vector<StPiece> pieces;
    if (!st_open_dir(dir, files, err) ||
        !st_expert_pieces(files, prefix ? prefix : "", fmt, D, I, layer0, layer1, n_experts,
                          pieces, err)) {
        set_error("slab_load: " + err);
        return 0;
    }
    long long off[6];
    Slab S;
    S.fmt = fmt;
    S.D = D;
    S.I = I;
    S.layer0 = layer0;
    S.layer1 = layer1;
    S.n_experts = n_experts;
    S.blob_bytes = mvllm_expert_geom(fmt, D, I, off);
    S.stride = (S.blob_bytes + 255) / 256 * 256;  // every blob 256-byte aligned
    const size_t n_blobs = (size_t)(layer1 - layer0) * n_experts;
    // spans in slab order, adjacent pieces merged when the file holds them back to back
    std::vector<Span> spans;
    for (size_t b = 0; b < n_blobs; ++b) {
        size_t dst = b * (size_t)S.stride;
        for (int k = 0; k < 6; ++k) {
            const StPiece &p = pieces[b * 6 + k];
            if (!spans.empty() && k > 0 && spans.back().file == p.file &&
                spans.back().off + spans.back().bytes == p.offset)
                spans.back().bytes += p.bytes;
            else
                spans.push_back({p.file, p.offset, p.bytes, dst});
            dst += p.bytes;
        }
    }
    std::vector<const void *> table(n_blobs);
    hipError_t e = hipMalloc(&S.base, n_blobs * (size_t)S.stride);
    if (e == hipSuccess)
        e = hipMalloc(&S.table, n_blobs * sizeof(void *));
    // the device blocks go back if anything below fails or throws
    struct Guard {
        Slab *s;
        ~Guard() {
            if (s) {
                if (s->base)
                    (void)hipFree(s->base);
                if (s->table)
                    (void)hipFree(s->table);
            }
        }
    } guard{&S};
    if (e != hipSuccess) {
        set_error(std::string("slab_load: hipMalloc: ") + hipGetErrorString(e));
        return 0;
    }
    for (size_t b = 0; b < n_blobs; ++b)
        table[b] = static_cast<char *>(S.base) + b * (size_t)S.stride;
    if (!stream_spans(files, spans, static_cast<char *>(S.base)) ||
        (e = hipMemcpy(S.table, table.data(), n_blobs * sizeof(void *),
                       hipMemcpyHostToDevice)) != hipSuccess) {
        if (e != hipSuccess)
            set_error(std::string("slab_load: hipMemcpy: ") + hipGetErrorString(e));
        return 0;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const long long h = g_next++;
    g_slabs[h] = S;
    guard.s = nullptr;
    return h;
}

// C entry: no exception (allocation failure included) crosses the boundary
extern "C" long long mvllm_hip_slab_load(const char *dir, const char *prefix, int fmt, int D,
                                         int I, int layer0, int layer1, int n_experts) {
    try {
        return slab_load_impl(dir, prefix, fmt, D, I, layer0, layer1, n_experts);
    } catch (const std::exception &x) {
        set_error(std::string("slab_load: ") + x.what());
    } catch (...) {
        set_error("slab_load: unknown exception");
    }
    return 0;
}

extern "C" int mvllm_hip_slab_info(long long h, void **base, void **table, long long *stride,
                                   long long *blob_bytes, int *n_blobs) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_slabs.find(h);
    if (it == g_slabs.end()) {
        set_error("slab_info: unknown handle");
        return 0;
    }
    const Slab &S = it->second;
    if (base)
        *base = S.base;
    if (table)
        *table = S.table;
    if (stride)
        *stride = S.stride;
    if (blob_bytes)
        *blob_bytes = S.blob_bytes;
    if (n_blobs)
        *n_blobs = (S.layer1 - S.layer0) * S.n_experts;
    return 1;
}

extern "C" int mvllm_hip_slab_free(long long h) {
    Slab S;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_slabs.find(h);
        if (it == g_slabs.end()) {
            set_error("slab_free: unknown handle");
            return 0;
        }
        S = it->second;
        g_slabs.erase(it);
    }
    // calls still reading the slab must finish first
    (void)hipDeviceSynchronize();
    (void)hipFree(S.base);
    (void)hipFree(S.table);
    return 1;
}
