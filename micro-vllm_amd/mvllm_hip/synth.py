"""Seeded synthetic moe_block workloads (the five benchmark configurations).

Inputs follow the benchmark definitions: activations N(0,1) rounded to bf16 and
passed as f32; int4-g64 codes uniform over all nibbles with bf16-valued scales
U(0.005, 0.02) stored as f32; MXFP4 codes uniform over all 16 e2m1 values with
ue8m0 bytes uniform in [118, 124]; per token k distinct experts (uniform, or
Zipf(1.1) popularity over a seeded permutation via Gumbel top-k); combine weights
are a softmax of N(0,1) logits.  The batched moe_block arguments come from the
segment builder (mvllm_moe_segments), which reproduces the engine's gather loop.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import ACT_CLAMP_SWIGLU, ACT_SILU, ACT_SITU, segments

SEED_BASE = 20261201

CONFIGS = {
    # name: shapes, format, activation (act, a, b), routing
    "c0": dict(D=1024, I=512, E=8, k=2, T=1, fmt=4, act=ACT_CLAMP_SWIGLU, a=7.0, b=0.0,
               routing="uniform", desc="tiny GLM-style int4-g64, T=1"),
    "c1": dict(D=2048, I=1024, E=64, k=8, T=16, fmt=4, act=ACT_SILU, a=0.0, b=0.0,
               routing="uniform", desc="OLMoE-shape int4-g64 decode"),
    "c2": dict(D=7168, I=2048, E=384, k=8, T=1, fmt=7, act=ACT_SITU, a=4.0, b=25.0,
               routing="uniform", desc="K3-style MXFP4 decode"),
    "c3": dict(D=6144, I=2048, E=256, k=8, T=512, fmt=4, act=ACT_CLAMP_SWIGLU, a=7.0, b=0.0,
               routing="uniform", desc="GLM-style int4-g64 prefill"),
    "c4": dict(D=7168, I=2048, E=384, k=8, T=2048, fmt=7, act=ACT_SITU, a=4.0, b=25.0,
               routing="zipf", desc="K3-style MXFP4 prefill, Zipf(1.1)"),
}


def bf16_round(x):
    """Round-to-nearest-even to bf16, returned as f32 (Inf/NaN truncated)."""
    x = np.ascontiguousarray(x, np.float32)
    b = x.view(np.uint32).copy()
    fin = (b & 0x7F800000) != 0x7F800000
    b[fin] = b[fin] + np.uint32(0x7FFF) + ((b[fin] >> 16) & 1)
    return (b & np.uint32(0xFFFF0000)).view(np.float32)


def routing(rng, T, E, k, kind="uniform", zipf_s=1.1):
    """-> idx [T,k] int32 (distinct per token), wt [T,k] f32 (softmax of N(0,1))."""
    if kind == "uniform":
        keys = rng.random((T, E))
    else:
        perm = rng.permutation(E)
        p = np.empty(E)
        p[perm] = (np.arange(1, E + 1, dtype=np.float64)) ** (-zipf_s)
        g = -np.log(-np.log(rng.random((T, E))))
        keys = np.log(p)[None, :] + g
    idx = np.argsort(-keys, axis=1, kind="stable")[:, :k].astype(np.int32)
    logits = rng.standard_normal((T, k)).astype(np.float32)
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    wt = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, wt


def piece_shapes(fmt, D, I):
    """Shapes of (gate/up packed, gate/up scales, down packed, down scales)."""
    if fmt == 0:
        return (I, D), None, (D, I), None
    gq = 64 if fmt == 4 else 32
    return (I, (D + 1) // 2), (I, (D + gq - 1) // gq), (D, (I + 1) // 2), (D, (I + gq - 1) // gq)


def make_expert(rng, fmt, D, I):
    """One expert: dict gp, gs, up, us, dp, ds (numpy, reference layouts)."""
    pw, ps, dw, dsh = piece_shapes(fmt, D, I)
    ex = {}
    for m, (wsh, ssh) in (("g", (pw, ps)), ("u", (pw, ps)), ("d", (dw, dsh))):
        if fmt == 0:
            ex[m + "p"] = (rng.standard_normal(wsh) * 0.05).astype(np.float32)
            ex[m + "s"] = None
        elif fmt == 4:
            ex[m + "p"] = rng.integers(0, 256, size=wsh, dtype=np.uint8)
            ex[m + "s"] = bf16_round(rng.uniform(0.005, 0.02, size=ssh).astype(np.float32))
        else:
            ex[m + "p"] = rng.integers(0, 256, size=wsh, dtype=np.uint8)
            ex[m + "s"] = rng.integers(118, 125, size=ssh, dtype=np.uint8)
    return ex


def device_pool(torch, fmt, D, I, n_blobs, seed, geom):
    """n_blobs expert blobs in the reference layout, generated on the GPU with the same
    distributions as make_expert (codes uniform over all bytes; int4 scales U(0.005, 0.02)
    rounded to bf16 and stored as f32; ue8m0 bytes in [118, 124]).  geom = expert_geom's
    (bytes, offsets[6]).  Returns (pool [n_blobs, stride] uint8 on the device, stride)."""
    nbytes, off = geom
    stride = (nbytes + 255) // 256 * 256
    g = torch.Generator(device="cuda").manual_seed(seed)
    pool = torch.randint(0, 256, (n_blobs, stride), dtype=torch.uint8, device="cuda",
                         generator=g)
    gq = 64 if fmt == 4 else 32
    for oi, O, K in ((1, I, D), (3, I, D), (5, D, I)):  # scale pieces: (offset index, O, K)
        ns = O * ((K + gq - 1) // gq)
        o = int(off[oi])
        if fmt == 4:
            s = torch.empty((n_blobs, ns), dtype=torch.float32, device="cuda")
            s.uniform_(0.005, 0.02, generator=g)
            s = s.to(torch.bfloat16).to(torch.float32)  # bf16-valued scales stored as f32
            pool[:, o:o + 4 * ns] = s.view(torch.uint8).view(n_blobs, 4 * ns)
        else:
            pool[:, o:o + ns] = torch.randint(118, 125, (n_blobs, ns), dtype=torch.uint8,
                                              device="cuda", generator=g)
    return pool, stride


def blob_pieces(blob, fmt, D, I, off):
    """Host numpy views (gp, up, dp, gs, us, ds) of one expert blob (uint8 numpy)."""
    gq, sb = (64, 4) if fmt == 4 else (32, 1)

    def piece(oi, O, K, scale):
        o = int(off[oi])
        if scale:
            n = O * ((K + gq - 1) // gq)
            return blob[o:o + n * sb].view(np.float32 if fmt == 4 else np.uint8).reshape(O, -1)
        return blob[o:o + O * ((K + 1) // 2)].reshape(O, -1)
    return (piece(0, I, D, False), piece(2, I, D, False), piece(4, D, I, False),
            piece(1, I, D, True), piece(3, I, D, True), piece(5, D, I, True))


@dataclass
class Workload:
    name: str
    D: int
    I: int
    fmt: int
    act: int
    a: float
    b: float
    T: int
    x: np.ndarray              # [T, D] f32 (bf16-valued)
    idx: np.ndarray            # [T, k]
    wt: np.ndarray             # [T, k]
    nb: int
    eids: np.ndarray
    xoff: np.ndarray
    nr: np.ndarray
    rows: np.ndarray
    rw: np.ndarray
    xg: np.ndarray             # [sum nr, D] gathered rows
    experts: dict = field(default_factory=dict)  # eid -> expert dict

    def lists(self):
        """Per-expert pointer lists in segment order: (g, u, d, gs, us, ds)."""
        ex = [self.experts[int(e)] for e in self.eids]
        return ([e["gp"] for e in ex], [e["up"] for e in ex], [e["dp"] for e in ex],
                [e["gs"] for e in ex], [e["us"] for e in ex], [e["ds"] for e in ex])


def make_workload(name, T=None, seed=None, with_experts=True, **over):
    cfg = dict(CONFIGS[name])
    cfg.update(over)
    T = cfg["T"] if T is None else T
    seed = SEED_BASE + int(name[1:]) if seed is None else seed
    rng = np.random.default_rng(seed)
    D, I, E, k = cfg["D"], cfg["I"], cfg["E"], cfg["k"]
    x = bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    idx, wt = routing(rng, T, E, k, cfg["routing"])
    nb, eids, xoff, nr, rows, rw = segments(idx, wt, T, k, E)
    xg = np.ascontiguousarray(x[rows])
    experts = {}
    if with_experts:
        for e in eids:
            erng = np.random.default_rng([seed, int(e)])
            experts[int(e)] = make_expert(erng, cfg["fmt"], D, I)
    return Workload(name, D, I, cfg["fmt"], cfg["act"], cfg["a"], cfg["b"], T, x, idx, wt, nb,
                    eids, xoff, nr, rows, rw, xg, experts)
