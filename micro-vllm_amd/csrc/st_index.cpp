// st_index.cpp -- where each routed expert's six pieces lie in a safetensors container
// (host only, no device calls).
//
// A safetensors file is an 8-byte little-endian header length n, n bytes of JSON mapping
// tensor names to {dtype, shape, data_offsets: [begin, end]} (plus an optional
// "__metadata__" entry), then the data section; a tensor's bytes sit at file offset
// 8 + n + begin (src/io/safetensors.cpp:45-154, st_file_offset in
// src/io/safetensors.hpp:38-41).  A directory's containers are every regular file whose
// name ends in ".safetensors", in name order, and a name resolves to the first file that
// holds it (st_open_dir / st_find_dir, src/io/safetensors.cpp:183-235, 310-317).
//
// The expert pieces, per family:
//   fmt 4 (GLM, src/model/glm53.cpp:171-174, 1829-1871):
//     <prefix>layers.<L>.mlp.experts.<e>.{gate,up,down}_proj.weight      U8/I8 codes
//     <prefix>layers.<L>.mlp.experts.<e>.{gate,up,down}_proj.weight.qs   f32 scales
//   fmt 7 (K3, src/model/kimi_k3.cpp:211-212, 1881-1934):
//     <prefix>model.layers.<L>.block_sparse_moe.experts.<e>.w{1,2,3}.weight_{packed,scale}
// in blob order (gate_p gate_s up_p up_s down_p down_s for GLM, w1p w1s w2p w2s w3p w3s
// for K3), each piece's byte count checked against the blob geometry.
#include "../../include/mvllm_hip.h"

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include "st_index.hpp"

namespace mvllm_hip {
namespace {

// ---- a JSON reader for safetensors headers -------------------------------------------
// Objects, arrays, strings (with escapes), numbers, true / false / null.  Only what the
// header needs is kept: per tensor its dtype, shape and data offsets.

struct JReader {
    const char *p, *end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r'))
            ++p;
    }
    bool fail(const char *what) {
        if (err.empty())
            err = what;
        return false;
    }
    bool lit(const char *s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end - p) < n || std::memcmp(p, s, n) != 0)
            return fail("bad literal");
        p += n;
        return true;
    }
    static void utf8(std::string &o, unsigned cp) {
        if (cp < 0x80) {
            o += (char)cp;
        } else if (cp < 0x800) {
            o += (char)(0xc0 | (cp >> 6));
            o += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            o += (char)(0xe0 | (cp >> 12));
            o += (char)(0x80 | ((cp >> 6) & 0x3f));
            o += (char)(0x80 | (cp & 0x3f));
        } else {
            o += (char)(0xf0 | (cp >> 18));
            o += (char)(0x80 | ((cp >> 12) & 0x3f));
            o += (char)(0x80 | ((cp >> 6) & 0x3f));
            o += (char)(0x80 | (cp & 0x3f));
        }
    }
    bool hex4(unsigned &v) {
        if (end - p < 4)
            return fail("short \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9')
                v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f')
                v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F')
                v |= (unsigned)(c - 'A' + 10);
            else
                return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string &o) {
        ws();
        if (p >= end || *p != '"')
            return fail("expected a string");
        ++p;
        o.clear();
        while (p < end && *p != '"') {
            const unsigned char c = (unsigned char)*p++;
            if (c < 0x20)
                return fail("control character in a string");
            if (c != '\\') {
                o += (char)c;
                continue;
            }
            if (p >= end)
                return fail("unterminated escape");
            const char e = *p++;
            switch (e) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                unsigned cp;
                if (!hex4(cp))
                    return false;
                if (cp >= 0xd800 && cp < 0xdc00) {  // surrogate pair
                    unsigned lo;
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u')
                        return fail("lone surrogate");
                    p += 2;
                    if (!hex4(lo) || lo < 0xdc00 || lo >= 0xe000)
                        return fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                }
                utf8(o, cp);
                break;
            }
            default:
                return fail("bad escape");
            }
        }
        if (p >= end)
            return fail("unterminated string");
        ++p;
        return true;
    }
    // an integer (the only numbers a header holds); other numbers are skipped with ok=false
    bool num(long long &v, bool &integral) {
        ws();
        const char *s = p;
        if (p < end && *p == '-')
            ++p;
        if (p >= end || !(*p >= '0' && *p <= '9'))
            return fail("expected a number");
        while (p < end && *p >= '0' && *p <= '9')
            ++p;
        integral = true;
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
            integral = false;
            while (p < end && (std::strchr("0123456789.eE+-", *p) != nullptr))
                ++p;
        }
        if (integral) {
            // digits accumulated with an explicit bound: no library call that throws
            const bool neg = *s == '-';
            const unsigned long long lim =
                neg ? (unsigned long long)LLONG_MAX + 1ull : (unsigned long long)LLONG_MAX;
            unsigned long long a = 0;
            for (const char *d = neg ? s + 1 : s; d < p; ++d) {
                const unsigned dig = (unsigned)(*d - '0');
                if (a > (lim - dig) / 10ull)
                    return fail("integer out of range");
                a = a * 10ull + dig;
            }
            v = neg ? (a == (unsigned long long)LLONG_MAX + 1ull ? LLONG_MIN : -(long long)a)
                    : (long long)a;
        }
        return true;
    }
    bool skip_value(int depth = 0) {
        if (depth > 64)
            return fail("nesting too deep");
        ws();
        if (p >= end)
            return fail("unexpected end");
        if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            ++p;
            ws();
            if (p < end && *p == close) {
                ++p;
                return true;
            }
            for (;;) {
                if (obj) {
                    std::string k;
                    if (!str(k))
                        return false;
                    ws();
                    if (p >= end || *p != ':')
                        return fail("expected ':'");
                    ++p;
                }
                if (!skip_value(depth + 1))
                    return false;
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == close) {
                    ++p;
                    return true;
                }
                return fail("expected ',' or a closing bracket");
            }
        }
        if (*p == '"') {
            std::string s;
            return str(s);
        }
        if (*p == 't')
            return lit("true");
        if (*p == 'f')
            return lit("false");
        if (*p == 'n')
            return lit("null");
        long long v;
        bool in;
        return num(v, in);
    }
    // [int, int, ...]
    bool int_array(std::vector<long long> &out) {
        ws();
        if (p >= end || *p != '[')
            return fail("expected an array");
        ++p;
        out.clear();
        ws();
        if (p < end && *p == ']') {
            ++p;
            return true;
        }
        for (;;) {
            long long v;
            bool in;
            if (!num(v, in))
                return false;
            if (!in)
                return fail("expected an integer");
            out.push_back(v);
            ws();
            if (p < end && *p == ',') {
                ++p;
                continue;
            }
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            return fail("expected ',' or ']'");
        }
    }
};

bool ends_with(const std::string &s, const char *suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

std::string join_path(const std::string &dir, const std::string &name) {
    if (dir.empty())
        return name;
    return dir.back() == '/' ? dir + name : dir + "/" + name;
}

bool pread_all(int fd, void *dst, size_t n, off_t off) {
    char *d = static_cast<char *>(dst);
    while (n) {
        const ssize_t r = ::pread(fd, d, n, off);
        if (r < 0 && errno == EINTR)
            continue;
        if (r <= 0)
            return false;
        d += r;
        n -= (size_t)r;
        off += r;
    }
    return true;
}

}  // namespace

bool st_parse_header(const char *text, size_t n, std::vector<StEntry> &out, std::string &err) {
    JReader J{text, text + n, {}};
    out.clear();
    J.ws();
    if (J.p >= J.end || *J.p != '{') {
        err = "safetensors header is not an object";
        return false;
    }
    ++J.p;
    J.ws();
    if (J.p < J.end && *J.p == '}') {
        ++J.p;
        return true;
    }
    for (;;) {
        std::string name;
        if (!J.str(name))
            break;
        J.ws();
        if (J.p >= J.end || *J.p != ':') {
            J.fail("expected ':'");
            break;
        }
        ++J.p;
        if (name == "__metadata__") {
            if (!J.skip_value())
                break;
        } else {
            J.ws();
            if (J.p >= J.end || *J.p != '{') {
                err = "tensor entry is not an object: " + name;
                return false;
            }
            ++J.p;
            StEntry t;
            t.name = name;
            bool has_dtype = false, has_shape = false, has_off = false;
            J.ws();
            if (J.p < J.end && *J.p == '}') {
                ++J.p;
            } else {
                for (;;) {
                    std::string k;
                    if (!J.str(k))
                        break;
                    J.ws();
                    if (J.p >= J.end || *J.p != ':') {
                        J.fail("expected ':'");
                        break;
                    }
                    ++J.p;
                    if (k == "dtype") {
                        J.ws();
                        if (J.p < J.end && *J.p == '"') {
                            if (!J.str(t.dtype))
                                break;
                            has_dtype = true;
                        } else if (!J.skip_value()) {
                            break;
                        }
                    } else if (k == "shape") {
                        J.ws();
                        if (J.p < J.end && *J.p == '[') {
                            if (!J.int_array(t.shape))
                                break;
                            has_shape = true;
                        } else if (!J.skip_value()) {
                            break;
                        }
                    } else if (k == "data_offsets") {
                        std::vector<long long> o;
                        J.ws();
                        if (J.p < J.end && *J.p == '[') {
                            if (!J.int_array(o))
                                break;
                            if (o.size() == 2 && o[0] >= 0 && o[1] >= 0) {
                                t.begin = (uint64_t)o[0];
                                t.end = (uint64_t)o[1];
                                has_off = true;
                            }
                        } else if (!J.skip_value()) {
                            break;
                        }
                    } else if (!J.skip_value()) {
                        break;
                    }
                    J.ws();
                    if (J.p < J.end && *J.p == ',') {
                        ++J.p;
                        continue;
                    }
                    if (J.p < J.end && *J.p == '}') {
                        ++J.p;
                        break;
                    }
                    J.fail("expected ',' or '}'");
                    break;
                }
            }
            if (!J.err.empty())
                break;
            if (!has_dtype) {
                err = "missing dtype: " + name;
                return false;
            }
            if (!has_shape) {
                err = "missing shape: " + name;
                return false;
            }
            if (!has_off) {
                err = "bad data_offsets: " + name;
                return false;
            }
            if (t.end < t.begin) {
                err = "data_offsets inverted: " + name;
                return false;
            }
            out.push_back(std::move(t));
        }
        J.ws();
        if (J.p < J.end && *J.p == ',') {
            ++J.p;
            continue;
        }
        if (J.p < J.end && *J.p == '}') {
            ++J.p;
            break;
        }
        J.fail("expected ',' or '}'");
        break;
    }
    if (!J.err.empty()) {
        err = "safetensors header: " + J.err;
        return false;
    }
    return true;
}

bool st_open_file(const std::string &path, StFileIdx &f, std::string &err) {
    f = StFileIdx();
    f.path = path;
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        err = "open(" + path + "): " + std::strerror(errno);
        return false;
    }
    struct stat st {};
    const bool have_size = ::fstat(fd, &st) == 0;
    f.size = have_size ? (uint64_t)st.st_size : 0;
    unsigned char hs[8];
    if (!pread_all(fd, hs, 8, 0)) {
        ::close(fd);
        err = "read(" + path + "): short header";
        return false;
    }
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i)
        n = (n << 8) | hs[i];
    // the safetensors format's own bound on the header (100 MB)
    if (n == 0 || n > 100ull * 1000ull * 1000ull) {
        ::close(fd);
        err = "invalid safetensors header_size";
        return false;
    }
    f.data_origin = 8 + n;
    if (have_size && f.data_origin > f.size) {
        ::close(fd);
        err = "safetensors header exceeds file size";
        return false;
    }
    std::string text(n, '\0');
    const bool ok = pread_all(fd, &text[0], n, 8);
    ::close(fd);
    if (!ok) {
        err = "read(" + path + "): short header";
        return false;
    }
    std::vector<StEntry> ents;
    if (!st_parse_header(text.data(), text.size(), ents, err))
        return false;
    f.tensors = std::move(ents);
    for (size_t i = 0; i < f.tensors.size(); ++i)
        f.index.emplace(f.tensors[i].name, i);
    return true;
}

bool st_open_dir(const std::string &dir, std::vector<StFileIdx> &out, std::string &err) {
    out.clear();
    DIR *d = ::opendir(dir.c_str());
    if (!d) {
        err = "opendir(" + dir + "): " + std::strerror(errno);
        return false;
    }
    std::vector<std::string> paths;
    while (struct dirent *e = ::readdir(d)) {
        const std::string name = e->d_name;
        if (name == "." || name == ".." || !ends_with(name, ".safetensors"))
            continue;
        const std::string full = join_path(dir, name);
        struct stat st {};
        if (::stat(full.c_str(), &st) != 0 || S_ISDIR(st.st_mode))
            continue;
        paths.push_back(full);
    }
    ::closedir(d);
    std::sort(paths.begin(), paths.end());
    for (const auto &p : paths) {
        StFileIdx f;
        if (!st_open_file(p, f, err)) {
            out.clear();
            return false;
        }
        out.push_back(std::move(f));
    }
    return true;
}

// The name of piece k (blob order) of expert e in layer L.
std::string expert_piece_name(int fmt, const std::string &prefix, int L, int e, int k) {
    static const char *glm[6] = {"gate_proj.weight", "gate_proj.weight.qs", "up_proj.weight",
                                 "up_proj.weight.qs", "down_proj.weight", "down_proj.weight.qs"};
    static const char *mats[3] = {"w1", "w2", "w3"};
    static const char *half[2] = {"packed", "scale"};
    if (fmt == 4)
        return prefix + "layers." + std::to_string(L) + ".mlp.experts." + std::to_string(e) +
               "." + glm[k];
    return prefix + "model.layers." + std::to_string(L) + ".block_sparse_moe.experts." +
           std::to_string(e) + "." + mats[k / 2] + ".weight_" + half[k & 1];
}

// Byte count of each piece in blob order.
bool expert_piece_bytes(int fmt, int D, int I, long long want[6]) {
    long long off[6];
    const long long total = mvllm_expert_geom(fmt, D, I, off);
    if (total < 0)
        return false;
    // blob order == name order for both families; the geometry's offsets are indexed
    // gate_p gate_s up_p up_s down_p down_s
    long long start[6];
    if (fmt == 4) {
        for (int k = 0; k < 6; ++k)
            start[k] = off[k];
    } else {  // w1p w1s w2p w2s w3p w3s = gate_p gate_s down_p down_s up_p up_s
        start[0] = off[0];
        start[1] = off[1];
        start[2] = off[4];
        start[3] = off[5];
        start[4] = off[2];
        start[5] = off[3];
    }
    for (int k = 0; k < 6; ++k)
        want[k] = (k < 5 ? start[k + 1] : total) - start[k];
    return true;
}

bool st_expert_pieces(const std::vector<StFileIdx> &files, const std::string &prefix, int fmt,
                      int D, int I, int layer0, int layer1, int n_experts,
                      std::vector<StPiece> &out, std::string &err) {
    out.clear();
    long long want[6];
    if ((fmt != 4 && fmt != 7) || !expert_piece_bytes(fmt, D, I, want) || layer1 <= layer0 ||
        n_experts < 1) {
        err = "st_expert_pieces: bad arguments";
        return false;
    }
    auto find = [&](const std::string &n, int &fi) -> const StEntry * {
        for (size_t i = 0; i < files.size(); ++i) {
            auto it = files[i].index.find(n);
            if (it != files[i].index.end()) {
                fi = (int)i;
                return &files[i].tensors[it->second];
            }
        }
        return nullptr;
    };
    const char *fam = fmt == 4 ? "glm53" : "k3 MXFP4";
    if (fmt == 4) {
        // GLM streams U8 / I8 containers only (src/model/glm53.cpp:1829): a float
        // checkpoint has to be converted first
        int fi;
        const StEntry *probe = find(expert_piece_name(fmt, prefix, layer0, 0, 0), fi);
        if (probe && probe->dtype != "U8" && probe->dtype != "I8") {
            err = "glm53 f32 expert checkpoint: use convert_glm53.py or a U8 container";
            return false;
        }
    }
    out.reserve((size_t)(layer1 - layer0) * n_experts * 6);
    for (int L = layer0; L < layer1; ++L)
        for (int e = 0; e < n_experts; ++e)
            for (int k = 0; k < 6; ++k) {
                int fi = -1;
                const StEntry *t = find(expert_piece_name(fmt, prefix, L, e, k), fi);
                if (!t || (long long)(t->end - t->begin) != want[k]) {
                    err = std::string(fam) + " expert pieces missing or wrong size at L" +
                          std::to_string(L) + " E" + std::to_string(e);
                    out.clear();
                    return false;
                }
                StPiece p;
                p.file = fi;
                p.offset = files[fi].data_origin + t->begin;
                p.bytes = (uint64_t)want[k];
                if (files[fi].size && p.offset + p.bytes > files[fi].size) {
                    err = std::string(fam) + " expert piece past the end of " + files[fi].path +
                          " at L" + std::to_string(L) + " E" + std::to_string(e);
                    out.clear();
                    return false;
                }
                out.push_back(p);
            }
    return true;
}

}  // namespace mvllm_hip

namespace {
int expert_pieces_impl(const char *dir, const char *prefix, int fmt, int D, int I, int layer0,
                       int layer1, int n_experts, int *file, long long *offset,
                       long long *bytes, char *paths, long long paths_cap, char *err,
                       long long err_cap) {
    using namespace mvllm_hip;
    std::string e;
    std::vector<StFileIdx> files;
    std::vector<StPiece> pieces;
    auto put_err = [&](const std::string &s) {
        if (err && err_cap > 0) {
            const size_t n = std::min((size_t)err_cap - 1, s.size());
            std::memcpy(err, s.data(), n);
            err[n] = '\0';
        }
    };
    if (!dir) {
        put_err("st_expert_pieces: null dir");
        return -1;
    }
    if (!st_open_dir(dir, files, e) ||
        !st_expert_pieces(files, prefix ? prefix : "", fmt, D, I, layer0, layer1, n_experts,
                          pieces, e)) {
        put_err(e);
        return -1;
    }
    for (size_t i = 0; i < pieces.size(); ++i) {
        if (file)
            file[i] = pieces[i].file;
        if (offset)
            offset[i] = (long long)pieces[i].offset;
        if (bytes)
            bytes[i] = (long long)pieces[i].bytes;
    }
    if (paths && paths_cap > 0) {
        std::string all;
        for (const auto &f : files)
            all += f.path + "\n";
        if ((long long)all.size() >= paths_cap) {
            put_err("st_expert_pieces: path buffer too small");
            return -1;
        }
        std::memcpy(paths, all.c_str(), all.size() + 1);
    }
    put_err("");
    return (int)files.size();
}
}  // namespace

// C entry: no exception (allocation failure included) crosses the boundary
extern "C" int mvllm_st_expert_pieces(const char *dir, const char *prefix, int fmt, int D, int I,
                                      int layer0, int layer1, int n_experts, int *file,
                                      long long *offset, long long *bytes, char *paths,
                                      long long paths_cap, char *err, long long err_cap) {
    try {
        return expert_pieces_impl(dir, prefix, fmt, D, I, layer0, layer1, n_experts, file,
                                  offset, bytes, paths, paths_cap, err, err_cap);
    } catch (const std::exception &x) {
        if (err && err_cap > 0)
            std::snprintf(err, (size_t)err_cap, "st_expert_pieces: %s", x.what());
    } catch (...) {
        if (err && err_cap > 0)
            std::snprintf(err, (size_t)err_cap, "st_expert_pieces: unknown exception");
    }
    return -1;
}
