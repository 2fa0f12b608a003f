// st_index.hpp -- safetensors container index and the routed experts' piece locations
// (host only).  See st_index.cpp.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace mvllm_hip {

struct StEntry {
    std::string name, dtype;
    std::vector<long long> shape;
    uint64_t begin = 0, end = 0;  // within the data section
};

struct StFileIdx {
    std::string path;
    uint64_t size = 0, data_origin = 0;  // data section at file offset data_origin
    std::vector<StEntry> tensors;
    std::unordered_map<std::string, size_t> index;
};

// One expert piece: file index, absolute file offset, byte count.
struct StPiece {
    int file = -1;
    uint64_t offset = 0, bytes = 0;
};

bool st_parse_header(const char *text, size_t n, std::vector<StEntry> &out, std::string &err);
bool st_open_file(const std::string &path, StFileIdx &f, std::string &err);
bool st_open_dir(const std::string &dir, std::vector<StFileIdx> &out, std::string &err);
std::string expert_piece_name(int fmt, const std::string &prefix, int L, int e, int k);
bool expert_piece_bytes(int fmt, int D, int I, long long want[6]);
// Six pieces per (layer, expert), layers [layer0, layer1) outer, experts inner, pieces in
// blob order.
bool st_expert_pieces(const std::vector<StFileIdx> &files, const std::string &prefix, int fmt,
                      int D, int I, int layer0, int layer1, int n_experts,
                      std::vector<StPiece> &out, std::string &err);

}  // namespace mvllm_hip
