"""Float64 brute-force restatement of the moe_block maths, written from the
definitions (not from the oracle's C), used to pin the oracle and to bound the
GPU error.  Dequantization here is exact (it is exact in f32 as well)."""
from __future__ import annotations

import numpy as np

E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def unpack_nibbles(packed, K):
    """[O, ceil(K/2)] bytes -> [O, K] nibbles; the low nibble is the even index."""
    p = np.asarray(packed, np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), np.uint8)
    out[:, 0::2] = p & 15
    out[:, 1::2] = p >> 4
    return out[:, :K]


def dequant(fmt, packed, scales, K):
    """Exact dequantized weights [O, K] in f32 (as the reference's inner loop forms them)."""
    if fmt == 0:
        return np.asarray(packed, np.float32)
    n = unpack_nibbles(packed, K)
    kk = np.arange(K)
    if fmt == 4:
        s = np.asarray(scales, np.float32)[:, kk // 64]
        return (n.astype(np.float32) - np.float32(8)) * s
    e = np.asarray(scales, np.uint8)[:, kk // 32].astype(np.uint32)
    s = (e << np.uint32(23)).view(np.float32)  # 0 -> +0, 255 -> +inf
    with np.errstate(invalid="ignore", over="ignore"):
        return E2M1[n] * s


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def act64(act, g, u, a, b):
    g = g.astype(np.float64)
    u = u.astype(np.float64)
    if act == 1:
        if a > 0:
            g = np.minimum(g, a)
            u = np.clip(u, -a, a)
        return g * sigmoid(g) * u
    if act == 2:
        return a * np.tanh(g / a) * sigmoid(g) * b * np.tanh(u / b)
    return g * sigmoid(g) * u


def moe_block64(nb, D, I, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S, act, a, b):
    """Returns the f64 result of out + contributions (out is not modified)."""
    res = np.array(out, np.float64, copy=True)
    base = 0
    for e in range(nb):
        n = int(nr[e])
        if n <= 0:
            continue
        ok = I >= 1 and g is not None and u is not None and d is not None and \
            g[e] is not None and u[e] is not None and d[e] is not None
        if ok and fmt in (4, 7):
            ok = gs is not None and us is not None and ds is not None and \
                gs[e] is not None and us[e] is not None and ds[e] is not None
        if not ok:
            base += n
            continue
        xe = np.asarray(xg, np.float64)[int(xoff[e]):int(xoff[e]) + n]
        Wg = dequant(fmt, g[e], None if fmt == 0 else gs[e], D).astype(np.float64)
        Wu = dequant(fmt, u[e], None if fmt == 0 else us[e], D).astype(np.float64)
        Wd = dequant(fmt, d[e], None if fmt == 0 else ds[e], I).astype(np.float64)
        h = act64(act, xe @ Wg.T, xe @ Wu.T, a, b)
        y = h @ Wd.T
        if rows is not None and rw is not None:
            for r in range(n):
                dst = int(rows[base + r])
                if dst < 0 or (S > 0 and dst >= S):
                    continue
                res[dst] += float(rw[base + r]) * y[r]
        base += n
    return res


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))
