"""Random moe_block argument sets for parity tests (numpy, self-contained)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def expert_arrays(rng, fmt, D, I, scale_lo=0.005, scale_hi=0.02, e_lo=118, e_hi=124):
    gq = 64 if fmt == 4 else 32

    def mat(O, K):
        if fmt == 0:
            return (rng.standard_normal((O, K)) * 0.05).astype(np.float32), None
        p = rng.integers(0, 256, size=(O, (K + 1) // 2), dtype=np.uint8)
        ns = (K + gq - 1) // gq
        if fmt == 4:
            s = rng.uniform(scale_lo, scale_hi, size=(O, ns)).astype(np.float32)
        else:
            s = rng.integers(e_lo, e_hi + 1, size=(O, ns), dtype=np.uint8)
        return p, s

    gp, gs = mat(I, D)
    up, us = mat(I, D)
    dp, ds = mat(D, I)
    return dict(gp=gp, gs=gs, up=up, us=us, dp=dp, ds=ds)


@dataclass
class Case:
    nb: int
    D: int
    I: int
    fmt: int
    g: list
    u: list
    d: list
    gs: list
    us: list
    ds: list
    xg: np.ndarray
    xoff: np.ndarray
    nr: np.ndarray
    rows: np.ndarray
    rw: np.ndarray
    out: np.ndarray
    S: int
    act: int
    a: float
    b: float

    def args(self, out=None):
        return (self.nb, self.D, self.I, self.fmt, self.g, self.u, self.d, self.gs, self.us,
                self.ds, self.xg, self.xoff, self.nr, self.rows, self.rw,
                self.out.copy() if out is None else out, self.S)


def random_case(rng, fmt, D, I, nr, S, act=0, a=0.0, b=0.0, null_experts=(), invalid_rows=0,
                zero_out=False, x_scale=1.0):
    """nr: rows per expert (0 allowed).  Rows of xg are laid out expert after expert."""
    nb = len(nr)
    nr = np.asarray(nr, np.int32)
    total = int(nr.sum())
    ex = [expert_arrays(rng, fmt, D, I) for _ in range(nb)]
    g = [e["gp"] for e in ex]
    u = [e["up"] for e in ex]
    d = [e["dp"] for e in ex]
    gs = [e["gs"] for e in ex] if fmt else None
    us = [e["us"] for e in ex] if fmt else None
    ds = [e["ds"] for e in ex] if fmt else None
    for e in null_experts:
        g[e] = None
    xg = (rng.standard_normal((max(total, 1), D)) * x_scale).astype(np.float32)
    xoff = np.concatenate([[0], np.cumsum(nr)[:-1]]).astype(np.int32)
    rows = rng.integers(0, max(S, 1), size=max(total, 1)).astype(np.int32)
    if invalid_rows and total:
        bad = rng.choice(total, size=min(invalid_rows, total), replace=False)
        rows[bad] = np.where(rng.random(len(bad)) < 0.5, -1, max(S, 1) + 3)
    rw = rng.uniform(0.05, 1.0, size=max(total, 1)).astype(np.float32)
    out = np.zeros((max(S, 1), D), np.float32) if zero_out else \
        rng.standard_normal((max(S, 1), D)).astype(np.float32)
    return Case(nb, D, I, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S, act, a, b)
