"""The engine-side binding as compiled code (CPU test).

Every C++ block of INTEGRATION.md tagged // [binding:...] is extracted from the document
itself (so the text cannot drift from what is tested) and assembled into one program:
  * device selection in gpu::select (src/gpu/backend.cpp:92-113), the one-expert call
    site glm_expert_try_hip (src/model/glm53.cpp:135-153) and the coli= tag
    (src/model/glm53.cpp:407-413);
  * the one-call-per-layer site glm_moe_layer_hip replacing the per-expert loop
    (src/model/glm53.cpp:1938-1992);
  * the HBM tier's hooks in ExpertStore (slot allocation, the slot-rewrite hook) and the
    engine-side prefetch and REPIN forwarding over the store's public interface;
  * the GPU-resident layer (device routing, tier table, routed block) and the hip= info
    line (src/engine.cpp:498-523).
It is compiled with g++ against the reference's own headers, together with csrc/hip_ops.cpp,
the reference's src/io/file_io.cpp where it lies, and a temporary copy of its
src/store/expert_store.cpp with INTEGRATION.md's three edits applied (STORE_EDITS), linked
with libmvllm_hip.so, and run.  Without a device (this container) selection falls back,
the call sites return false ("use the host kernel"), the tag reads coli=off, and the store
runs on its own allocator: it reads back a file of expert blobs through four slots per
layer, the prefetch hook leases and releases, and the REPIN hook forwards its two
evictions.  backend_name() is "hip" either way.  Skipped where the reference tree is
absent (the GPU box).
"""
import os
import re
import subprocess
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"
LIB_DIR = os.path.join(ROOT, "micro-vllm_amd")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference tree absent")

HARNESS = r"""// Assembled by tests/test_binding.py from INTEGRATION.md's snippets.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <ostream>
#include <sstream>
#include <string>
#include <vector>

#include "core/types.hpp"
#include "gpu/coli_cuda.hpp"
#include "gpu/metal_ops.hpp"
#include "io/file_io.hpp"
#include "model/family.hpp"
#include "store/expert_store.hpp"
#include "hip_ops.hpp"
#include "mvllm_hip.h"

namespace mvllm {
// src/gpu/coli_cuda.cpp is not linked into this test: no CUDA device here.
namespace coli_cuda {
bool available() { return false; }
int available_device_count() { return 0; }
}  // namespace coli_cuda

namespace {
// glm53.cpp's file-local blob splitter, here from the library's expert geometry
// (the same six offsets, src/model/glm53.cpp:56-78,116-132).
bool glm_pack_int4_g64(const uint8_t *blob, int H, int O, const void **g, const void **u,
                       const void **d, const float **gs, const float **us, const float **ds) {
    long long off[6];
    if (!blob || mvllm_expert_geom(4, H, O, off) < 0)
        return false;
    *g = blob + off[0];
    *gs = reinterpret_cast<const float *>(blob + off[1]);
    *u = blob + off[2];
    *us = reinterpret_cast<const float *>(blob + off[3]);
    *d = blob + off[4];
    *ds = reinterpret_cast<const float *>(blob + off[5]);
    return true;
}
// gpu::select's backend state (src/gpu/backend.cpp)
struct Backend {};
Backend g_cpu;
Backend *g_active = &g_cpu;
bool g_hip_routed = false;
}  // namespace

Backend &select_device(Device want) {
@SELECT@
    g_active = &g_cpu;
    return *g_active;
}

@CALL@

@STORE_SLOTS@

@STORE_PREFETCH@

@STORE_REPIN@

@LAYER@

@ROUTED@

@HIP_INFO@

std::string coli_tag() {
    std::ostringstream os;
    os << "coli=";
@INFO@
    return os.str();
}
}  // namespace mvllm

using namespace mvllm;
static_assert(int(hip_ops::Act::Silu) == int(metal_ops::Act::Silu), "Act::Silu");
static_assert(int(hip_ops::Act::ClampSwiGLU) == int(metal_ops::Act::ClampSwiGLU), "Act::ClampSwiGLU");
static_assert(int(hip_ops::Act::Situ) == int(metal_ops::Act::Situ), "Act::Situ");

// The reference's ExpertStore (the patched copy) driving the tier through the hooks.
static int store_checks(bool up, int H, int O, const char *dir) {
    long long off[6];
    const long long eb = mvllm_expert_geom(4, H, O, off);
    const int L = 2, E = 6;
    const std::string path = std::string(dir) + "/experts.bin";
    {
        std::FILE *f = std::fopen(path.c_str(), "wb");
        if (!f)
            return 20;
        for (int b = 0; b < L * E; ++b) {
            std::vector<uint8_t> blob(static_cast<size_t>(eb), static_cast<uint8_t>(b + 1));
            std::fwrite(blob.data(), 1, blob.size(), f);
        }
        std::fclose(f);
    }
    ExpertStore store;
    std::string err;
    const int64_t slot = (eb + 4095) & ~int64_t{4095};
    if (store.open(L, E, eb, slot * 4 * L, err) != Status::Ok || store.slots_per_layer() != 4)
        return 21;
    for (int l = 0; l < L; ++l)
        for (int e = 0; e < E; ++e) {
            ExpertLoc loc;
            loc.key = {l, e};
            loc.path = path;
            loc.offset = static_cast<int64_t>(l * E + e) * eb;
            loc.bytes = eb;
            if (store.register_expert(loc, err) != Status::Ok)
                return 22;
        }
    // the next layer's experts: leased, handed to the tier (no device: refused), released
    const int ids[3] = {0, 1, 2};
    const int staged = hip_prefetch_layer(store, 0, ids, 3, err);
    if (up ? staged != 3 : staged != -1)
        return 23;
    // every lease released: six experts through four slots, two evictions
    for (int e = 0; e < E; ++e) {
        ExpertView v{};
        if (store.lookup({0, e}, v, err) != Status::Ok)
            return 24;
        const uint8_t want = static_cast<uint8_t>(e + 1);
        if (v.bytes != eb || v.data[0] != want || v.data[eb - 1] != want)
            return 25;
        store.release(v);
    }
    if (hip_drain_repin(store) != 2)
        return 26;
    // one call for a chunk of two tokens, top-2 (no device: false, nothing leased)
    const int idx[4] = {0, 3, 2, 3};
    const float wt[4] = {0.5f, 0.5f, 1.f, 0.f};
    std::vector<float> xs(2 * static_cast<size_t>(H), 0.25f), acc(2 * static_cast<size_t>(H), 0.f);
    if (glm_moe_layer_hip(store, 1, idx, wt, 2, 2, xs.data(), H, O, 7.f, acc.data(), err) != up)
        return 27;
    for (int e = 0; e < 4; ++e) {
        ExpertView v{};
        if (store.lookup({1, e}, v, err) != Status::Ok)
            return 28;
        store.release(v);
    }
    std::ostringstream info;
    hip_info_line(info);
    if (!up && !info.str().empty())
        return 29;
    store.close();
    std::remove(path.c_str());
    return 0;
}

int main(int argc, char **argv) {
    if (std::string(hip_ops::backend_name()) != "hip")
        return 1;
    if (parse_device("hip") != Device::Hip)
        return 2;
    select_device(parse_device("hip"));
    const bool up = hip_ops::available();
    if (up != g_hip_routed)
        return 3;
    // one GLM expert (H = 256, O = 256) whose codes are all 8, i.e. zero weights: y = 0
    const int H = 256, O = 256, S = 2;
    long long off[6];
    const long long bytes = mvllm_expert_geom(4, H, O, off);
    std::vector<uint8_t> blob(static_cast<size_t>(bytes), 0x88);
    for (int p = 1; p < 6; p += 2) {
        const long long end = p == 5 ? bytes : off[p + 1];
        for (long long b = off[p]; b + 4 <= end; b += 4) {
            const float one = 1.f;
            std::memcpy(&blob[static_cast<size_t>(b)], &one, 4);
        }
    }
    std::vector<float> x(S * H, 0.5f), y(S * H, 3.f);
    const bool ran = glm_expert_try_hip(y.data(), x.data(), S, blob.data(), H, O, 7.f);
    if (ran != up)
        return 4;
    if (ran)
        for (float v : y)
            if (v != 0.f)
                return 5;
    const std::string tag = coli_tag();
    if (tag != (up ? "coli=hip" : "coli=off"))
        return 6;
    const int st = store_checks(up, H, O, argc > 1 ? argv[1] : ".");
    if (st)
        return st;
    // the GPU-resident layer: compiled and linked (it needs device buffers to run)
    auto *routed = &k3_moe_layer_hip_dev;
    if (!routed)
        return 7;
    std::printf("%s routed=%d ran=%d name=%s store=ok\n", tag.c_str(), int(g_hip_routed),
                int(ran), hip_ops::backend_name());
    hip_ops::shutdown();
    return 0;
}
"""

# The three edits of INTEGRATION.md section 4, applied to a temporary copy of the
# reference's src/store/expert_store.cpp: (anchor, replacement) pairs.  The anchors are
# the calls and the signature the section names.
STORE_EDITS = [
    ("io::aligned_alloc_pages(", "hip_slot_alloc("),
    ("io::aligned_free_pages(", "hip_slot_free("),
    ("Status ExpertStore::load_into(int layer, int eid, Slot &slot, std::string &err) {",
     "Status ExpertStore::load_into(int layer, int eid, Slot &slot, std::string &err) {\n"
     "    hip_slot_rewrite(slot.base, expert_bytes_);"),
    ("namespace mvllm {",
     "namespace mvllm {\n"
     "void *hip_slot_alloc(size_t bytes);\n"
     "void hip_slot_free(void *p);\n"
     "void hip_slot_rewrite(const uint8_t *base, int64_t bytes);"),
]


def snippets():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    out = {}
    for block in re.findall(r"```cpp\n(.*?)```", text, re.S):
        m = re.match(r"// \[binding:(\w+)\]", block)
        if m:
            out[m.group(1)] = block
    return out


def patched_store(tmp_path):
    src = open(os.path.join(REF_SRC, "store", "expert_store.cpp")).read()
    for anchor, repl in STORE_EDITS:
        assert src.count(anchor) >= 1, anchor
        src = src.replace(anchor, repl, 1 if anchor.startswith(("Status", "namespace")) else -1)
    out = tmp_path / "expert_store_hip.cpp"
    out.write_text(src)
    return out


def test_binding_compiles_links_and_falls_back(tmp_path):
    s = snippets()
    need = {"select", "call", "info", "layer", "store_slots", "store_prefetch", "store_repin",
            "routed", "hip_info"}
    assert set(s) >= need, sorted(s)
    body = {k: textwrap.indent(v, "    ") for k, v in s.items()}
    src = HARNESS.replace("@SELECT@", body["select"]).replace("@INFO@", body["info"])
    for key in ("call", "layer", "store_slots", "store_prefetch", "store_repin", "routed",
                "hip_info"):
        src = src.replace("@%s@" % key.upper(), s[key])
    cpp = tmp_path / "engine_binding.cpp"
    cpp.write_text(src)
    store = patched_store(tmp_path)
    exe = tmp_path / "engine_binding"
    assert os.path.exists(os.path.join(LIB_DIR, "libmvllm_hip.so")), "build the library first"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-DMVLLM_WITH_HIP=1",
           f"-I{REF_SRC}", f"-iquote{REF_SRC}/store", f"-I{ROOT}/include",
           f"-I{ROOT}/micro-vllm_amd/csrc", str(cpp), str(store),
           os.path.join(REF_SRC, "io", "file_io.cpp"),
           f"{ROOT}/micro-vllm_amd/csrc/hip_ops.cpp", f"-L{LIB_DIR}", "-lmvllm_hip",
           f"-Wl,-rpath,{LIB_DIR}", "-Wl,-rpath-link,/opt/rocm/lib", "-lpthread", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr[-2000:])
    line = r.stdout.strip().splitlines()[-1]
    assert line.endswith("name=hip store=ok"), line
    assert line.startswith("coli=hip routed=1 ran=1") or line.startswith("coli=off routed=0 ran=0")
