// segments.cpp -- host integer work on the path: unique expert ids, per-expert row
// segments for one batched moe_block call, and expert blob geometry.
#include "../../include/mvllm_hip.h"

#include <algorithm>
#include <vector>

extern "C" int mvllm_moe_union_ids(const int *idx, int n_tok, int topk, int *out, int out_cap) {
    // src/model/ops.cpp:1082-1099: drop negative ids, sort, keep the first of each run
    if (!idx || !out || n_tok <= 0 || topk <= 0 || out_cap <= 0)
        return 0;
    std::vector<int> ids;
    ids.reserve(static_cast<size_t>(n_tok) * static_cast<size_t>(topk));
    for (size_t i = 0, n = static_cast<size_t>(n_tok) * topk; i < n; ++i)
        if (idx[i] >= 0)
            ids.push_back(idx[i]);
    std::sort(ids.begin(), ids.end());
    int cnt = 0;
    for (size_t i = 0; i < ids.size() && cnt < out_cap; ++i)
        if (cnt == 0 || ids[i] != out[cnt - 1])
            out[cnt++] = ids[i];
    return cnt;
}

extern "C" int mvllm_moe_segments(const int *idx, const float *wt, int n_tok, int topk,
                                  int *eids, int *xoff, int *nr, int *rows, float *rw,
                                  int cap_experts, int cap_rows, int *n_rows) {
    // src/model/glm53.cpp:1938-1971: for each unique expert (ascending) its rows are
    // the tokens, in order, whose weights for that expert sum (slot order, from 0)
    // to a non-zero value.  Bucketing by expert first keeps this O(T*k + nb).
    if (n_rows)
        *n_rows = 0;
    if (!idx || !wt || n_tok <= 0 || topk <= 0 || cap_experts <= 0)
        return 0;
    std::vector<int> uniq(static_cast<size_t>(cap_experts));
    const int nu = mvllm_moe_union_ids(idx, n_tok, topk, uniq.data(), cap_experts);
    // per token: its slots grouped by expert, summed in slot order
    std::vector<std::vector<std::pair<int, float>>> per_expert(static_cast<size_t>(nu));
    std::vector<std::pair<int, float>> tok;  // (expert id, wsum) for one token
    for (int c = 0; c < n_tok; ++c) {
        tok.clear();
        for (int t = 0; t < topk; ++t) {
            const int e = idx[static_cast<size_t>(c) * topk + t];
            if (e < 0)
                continue;
            auto it = std::find_if(tok.begin(), tok.end(),
                                   [e](const std::pair<int, float> &p) { return p.first == e; });
            if (it == tok.end())
                tok.emplace_back(e, 0.f + wt[static_cast<size_t>(c) * topk + t]);
            else
                it->second += wt[static_cast<size_t>(c) * topk + t];
        }
        for (const auto &p : tok) {
            const auto pos = std::lower_bound(uniq.begin(), uniq.begin() + nu, p.first);
            if (pos == uniq.begin() + nu || *pos != p.first)
                continue;  // beyond cap_experts
            if (p.second != 0.f)
                per_expert[static_cast<size_t>(pos - uniq.begin())].emplace_back(c, p.second);
        }
    }
    int j = 0;
    for (int ui = 0; ui < nu; ++ui) {
        eids[ui] = uniq[static_cast<size_t>(ui)];
        xoff[ui] = j;
        const auto &v = per_expert[static_cast<size_t>(ui)];
        if (j + static_cast<int>(v.size()) > cap_rows)
            return -1;
        for (const auto &p : v) {
            rows[j] = p.first;
            rw[j] = p.second;
            ++j;
        }
        nr[ui] = static_cast<int>(v.size());
    }
    if (n_rows)
        *n_rows = j;
    return nu;
}

extern "C" long long mvllm_expert_geom(int fmt, int D, int I, long long off[6]) {
    if (D <= 0 || I <= 0 || !off)
        return -1;
    long long pg, sg, pd, sd;  // gate/up packed + scales, down packed + scales
    if (fmt == 4) {
        // src/model/glm53.cpp:56-78 (both branches agree; this is the general one)
        pg = static_cast<long long>(I) * ((D + 1) / 2);
        sg = static_cast<long long>(I) * ((D + 63) / 64) * 4;
        pd = static_cast<long long>(D) * ((I + 1) / 2);
        sd = static_cast<long long>(D) * ((I + 63) / 64) * 4;
        // gate_p | gate_s | up_p | up_s | down_p | down_s
        off[0] = 0;
        off[1] = pg;
        off[2] = pg + sg;
        off[3] = 2 * pg + sg;
        off[4] = 2 * (pg + sg);
        off[5] = 2 * (pg + sg) + pd;
        return 2 * (pg + sg) + pd + sd;
    }
    if (fmt == 7) {
        // src/model/kimi_k3.cpp:83-102: w1p|w1s|w2p|w2s|w3p|w3s, gate=w1 down=w2 up=w3
        pg = static_cast<long long>(I) * ((D + 1) / 2);
        sg = static_cast<long long>(I) * ((D + 31) / 32);
        pd = static_cast<long long>(D) * ((I + 1) / 2);
        sd = static_cast<long long>(D) * ((I + 31) / 32);
        off[0] = 0;                  // w1p (gate)
        off[1] = pg;                 // w1s
        off[4] = pg + sg;            // w2p (down)
        off[5] = pg + sg + pd;       // w2s
        off[2] = pg + sg + pd + sd;  // w3p (up)
        off[3] = 2 * pg + sg + pd + sd;
        return 2 * (pg + sg) + pd + sd;
    }
    return -1;
}
