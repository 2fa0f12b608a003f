"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the checker.

How each oracle function is pinned:
  bf16_round            reference KATs (tests/test_host.cpp:8479-8483) + bit-exact vs _ref
  mx4_lut / mx4_scale   closed form over all codes + bit-exact vs _ref
  sigmoid / activations reference KATs (test_host.cpp:143-148) + bit-exact vs _ref
  matmul_f32/int4/mxfp4 identity KAT, f64 brute force (npref), bit-exact vs _ref
  dequant int4/mxfp4    exact closed form (npref.dequant), bit for bit
  moe_block             identity-weight KATs (test_host.cpp:2567-2602, 2626-2652, 2743-2789,
                        the last strengthened to its closed-form value), f64 brute force
                        including every skip rule, bit-exact vs _ref, golden fixtures
  moe_topk / union_ids  KATs (test_host.cpp:4916-4932), brute force, bit-exact vs _ref
  moe_segments          invariants + a direct restatement of the gather loop
  fp4_activation_qdq    KATs (test_host.cpp:8410-8413), closed-form invariants, brute-force
                        nearest-code search, bit-exact vs _ref
"""
import math

import numpy as np
import pytest

import npref
from cases import random_case

F32_EPS = 1.2e-7


# ---------------------------------------------------------------- reference KATs

def test_kat_activations(orc):
    assert abs(orc.situ_glu(0.0, 0.0, 4.0, 25.0)) <= 1e-6
    a = orc.clamped_swiglu(100.0, 1.0, 7.0)
    assert abs(a - 7.0 * orc.sigmoid(7.0) * 1.0) <= 1e-4


def test_kat_bf16(orc):
    assert orc.bf16_round(1.00390625) == 1.0
    assert orc.bf16_round(1.01171875) == 1.015625


def test_kat_matmul_identity(orc):
    y = orc.matmul(0, np.array([[3, 4]], np.float32), np.eye(2, dtype=np.float32))
    assert np.allclose(y, [[3, 4]], atol=1e-5)


def _identity_block(orc, act, a, b, x):
    eye = np.eye(4, dtype=np.float32)
    out = np.zeros((1, 4), np.float32)
    rc = orc.moe_block(1, 4, 4, 0, [eye], [eye], [eye], None, None, None,
                       np.asarray([x], np.float32), np.array([0], np.int32),
                       np.array([1], np.int32), np.array([0], np.int32),
                       np.array([1.0], np.float32), out, 1, act, a, b)
    return rc, out[0]


def test_kat_moe_block_identity_silu(orc):
    x = np.array([0.5, -0.25, 1.0, -1.0], np.float32)
    rc, out = _identity_block(orc, 0, 0.0, 0.0, x)
    assert rc == 1
    sig = 1 / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(out, x * sig * x, atol=1e-4)


def test_kat_moe_block_identity_clamp(orc):
    x = np.array([0.5, -0.25, 1.0, -1.0], np.float32)
    rc, out = _identity_block(orc, 1, 10.0, 0.0, x)
    assert rc == 1
    ref = [orc.clamped_swiglu(float(v), float(v), 10.0) for v in x]
    assert np.allclose(out, ref, atol=1e-4)


def test_kat_moe_block_mxfp4_situ_closed_form(orc):
    """Reference test packs 0.5*I (32x32) as MXFP4 and only checks finiteness; the
    packed form is code 6 (4.0) with ue8m0 124 (0.125) on the diagonal, so the exact
    output is y[0] = 0.5 * situ(0.5, 0.5), zeros elsewhere."""
    n = 32
    codes = np.zeros((n, n), np.uint8)
    np.fill_diagonal(codes, 6)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    sc = np.full((n, 1), 124, np.uint8)
    x = np.zeros((1, n), np.float32)
    x[0, 0] = 1.0
    out = np.zeros((1, n), np.float32)
    rc = orc.moe_block(1, n, n, 7, [packed], [packed], [packed], [sc], [sc], [sc], x,
                       np.array([0], np.int32), np.array([1], np.int32),
                       np.array([0], np.int32), np.array([1.0], np.float32), out, 1, 2, 4.0,
                       25.0)
    assert rc == 1
    v = 4 * math.tanh(0.5 / 4) * (1 / (1 + math.exp(-0.5))) * 25 * math.tanh(0.5 / 25)
    exp = np.zeros(n)
    exp[0] = 0.5 * v
    assert np.allclose(out[0], exp, rtol=1e-6, atol=1e-7)


def test_kat_topk_union(orc):
    sig = np.array([0.1, 0.4, 0.3, 0.2], np.float32)
    choice = np.array([0.1, 0.4, 10.3, 0.2], np.float32)
    k, idx, w = orc.moe_topk(choice, 2, sig)
    assert k == 2 and list(idx) == [2, 1]
    assert abs(w[0] - 0.3 / 0.7) < 1e-5 and abs(w[1] - 0.4 / 0.7) < 1e-5
    u = orc.moe_union_ids(np.array([3, 1, 3, 2, 1, -1], np.int32), 3, 2, 8)
    assert list(u) == [1, 2, 3]


def test_kat_native_act(orc):
    assert orc.e8m0_decode(0x7E) == 0.5
    assert orc.e8m0_decode(0x7F) == 1.0
    assert orc.e8m0_decode(0x80) == 2.0
    assert math.isnan(orc.e8m0_decode(0xFF))
    rc, out, sc, codes = orc.fp4_activation_qdq(np.ones(32, np.float32), 32)
    assert rc == 0 and sc[0] == 125 and np.all(out == 1.0)


# ---------------------------------------------------------------- closed forms

def test_mx4_codecs_closed_form(orc):
    lut = [orc.fn("mx4_lut")(n) for n in range(16)]
    assert np.array_equal(np.array(lut, np.float32).view(np.uint32), npref.E2M1.view(np.uint32))
    for s in range(256):
        v = orc.fn("mx4_scale")(s)
        if s == 0:
            assert v == 0.0 and math.copysign(1, v) == 1
        elif s == 255:
            assert math.isinf(v) and v > 0
        else:
            assert v == math.ldexp(1.0, s - 127)


@pytest.mark.parametrize("fmt,K", [(4, 128), (4, 100), (4, 33), (7, 96), (7, 50), (7, 31)])
def test_dequant_bit_exact_closed_form(orc, fmt, K):
    rng = np.random.default_rng(K + fmt)
    O = 7
    packed = rng.integers(0, 256, size=(O, (K + 1) // 2), dtype=np.uint8)
    if fmt == 4:
        scales = rng.uniform(-0.03, 0.03, size=(O, (K + 63) // 64)).astype(np.float32)
    else:
        scales = rng.integers(0, 256, size=(O, (K + 31) // 32), dtype=np.uint8)
    w = orc.dequant(fmt, packed, scales, O, K)
    exp = npref.dequant(fmt, packed, scales, K)
    assert np.array_equal(w.view(np.uint32), exp.view(np.uint32))


def test_kat_matmul_int8_row(orc):
    """quant::matmul_int8_row: the row scale multiplies the whole sum, once."""
    x = np.array([[1, 2, -1]], np.float32)
    q = np.array([[1, 0, 3], [0, -3, 127], [-127, 1, 0]], np.int8)
    s = np.array([0.5, 2.0, 0.25], np.float32)
    assert orc.matmul(8, x, q, s).tolist() == [[-1.0, -266.0, -31.25]]


@pytest.mark.parametrize("fmt", [0, 4, 7, 8])
def test_matmul_vs_f64(orc, fmt):
    rng = np.random.default_rng(11 + fmt)
    S, K, O = 3, 160, 24  # non-square: a transposed operand cannot pass
    x = rng.standard_normal((S, K)).astype(np.float32)
    if fmt == 0:
        w, s = rng.standard_normal((O, K)).astype(np.float32), None
    elif fmt == 4:
        w = rng.integers(0, 256, size=(O, K // 2), dtype=np.uint8)
        s = rng.uniform(0.005, 0.02, size=(O, (K + 63) // 64)).astype(np.float32)
    elif fmt == 7:
        w = rng.integers(0, 256, size=(O, K // 2), dtype=np.uint8)
        s = rng.integers(118, 125, size=(O, K // 32), dtype=np.uint8)
    else:
        w = rng.integers(-127, 128, size=(O, K), dtype=np.int8)
        s = rng.uniform(0.001, 0.01, size=O).astype(np.float32)
    y = orc.matmul(fmt, x, w, s)
    if fmt == 8:
        wd = w.astype(np.float64) * s.astype(np.float64)[:, None]
    else:
        wd = npref.dequant(fmt, w, s, K).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    assert npref.rel_err(y, ref) < 20 * K * F32_EPS / np.sqrt(K)


CASES = [
    # fmt, D, I, nr, S, act, a, b, null_experts, invalid_rows
    (4, 128, 64, [2, 0, 3, 1], 5, 1, 7.0, 0.0, (), 0),
    (4, 96, 80, [1, 2], 3, 0, 0.0, 0.0, (1,), 1),
    (4, 70, 33, [3], 4, 1, 0.0, 0.0, (), 0),      # odd sizes, clamp disabled
    (7, 96, 64, [2, 1, 2], 4, 2, 4.0, 25.0, (), 2),
    (7, 65, 31, [1, 1], 2, 2, 4.0, 25.0, (), 0),   # odd sizes
    (0, 40, 24, [2, 1], 3, 1, 3.0, 0.0, (0,), 0),
]


@pytest.mark.parametrize("case", CASES)
def test_moe_block_vs_f64(orc, case):
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    rng = np.random.default_rng(D * 7 + I)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    out = c.out.copy()
    assert orc.moe_block(*c.args(out), act, a, b) == 1
    ref = npref.moe_block64(*c.args(), act, a, b)
    assert npref.rel_err(out, ref) < 2e-5


def test_moe_block_validation(orc):
    rng = np.random.default_rng(3)
    c = random_case(rng, 4, 64, 64, [1], 1)
    base = c.args()
    out = c.out.copy()
    for bad in ({0: 0}, {1: 0}, {3: 5}, {3: 1}, {10: None}, {11: None}, {12: None}, {15: None}):
        args = list(base)
        args[15] = out
        for k, v in bad.items():
            args[k] = v
        assert orc.moe_block(*args, 0, 0.0, 0.0) == 0
    # Iinter < 1: experts skipped, returns 1, out untouched
    args = list(base)
    args[2] = 0
    o2 = c.out.copy()
    args[15] = o2
    assert orc.moe_block(*args, 0, 0.0, 0.0) == 1 and np.array_equal(o2, c.out)
    # rows == NULL: computes, writes nothing
    args = list(base)
    args[13] = None
    o3 = c.out.copy()
    args[15] = o3
    assert orc.moe_block(*args, 0, 0.0, 0.0) == 1 and np.array_equal(o3, c.out)


def test_topk_brute_force(orc):
    rng = np.random.default_rng(5)
    for _ in range(50):
        n = int(rng.integers(1, 40))
        k = int(rng.integers(1, n + 3))
        choice = rng.integers(-3, 4, size=n).astype(np.float32)  # many ties
        mix = rng.uniform(-0.2, 1.0, size=n).astype(np.float32)
        kk, idx, w = orc.moe_topk(choice, k, mix)
        order = sorted(range(n), key=lambda i: (-float(choice[i]), i))[:min(k, n)]
        assert kk == min(k, n) and list(idx) == order
        ww = np.maximum(mix[order], 0).astype(np.float32)
        s = np.float32(0)
        for v in ww:
            s = np.float32(s + v)
        exp = ww / s if s > 0 else np.full(len(ww), np.float32(1) / np.float32(len(ww)))
        assert np.array_equal(w, exp.astype(np.float32))


def test_topk_batch_matches_per_token(orc):
    """The one-call batch (timed by bench.py's routing baseline) gives each token's
    moe_topk, in both libraries."""
    rng = np.random.default_rng(6)
    T, n, k = 19, 33, 5
    choice = rng.integers(-3, 4, size=(T, n)).astype(np.float32)
    mix = rng.uniform(-0.2, 1.0, size=(T, n)).astype(np.float32)
    import oracle
    for lib in [orc] + ([oracle.CpuMoe("ref")] if oracle.have_ref() else []):
        kk, idx, w = lib.moe_topk_batch(choice, k, mix)
        assert kk == k
        for t in range(T):
            _, i1, w1 = orc.moe_topk(choice[t], k, mix[t])
            assert np.array_equal(idx[t], i1) and np.array_equal(_bits(w[t]), _bits(w1))


def test_segments_invariants(orc):
    rng = np.random.default_rng(9)
    T, E, k = 37, 12, 4
    idx = rng.integers(-1, E, size=(T, k)).astype(np.int32)  # duplicates and -1 allowed
    wt = rng.uniform(0, 1, size=(T, k)).astype(np.float32)
    wt[rng.random((T, k)) < 0.1] = 0.0
    nb, eids, xoff, nr, rows, rw = orc.moe_segments(idx, wt, T, k, E)
    assert list(eids) == sorted(set(idx[idx >= 0].tolist()))
    assert np.all(np.diff(eids) > 0) and xoff[0] == 0
    assert np.array_equal(xoff[1:], np.cumsum(nr)[:-1])
    for i, e in enumerate(eids):
        seg = slice(xoff[i], xoff[i] + nr[i])
        toks = rows[seg]
        assert np.all(np.diff(toks) > 0)  # tokens ascending within an expert
        for c in range(T):
            ws = np.float32(0)
            for t in range(k):
                if idx[c, t] == e:
                    ws = np.float32(ws + wt[c, t])
            if ws != 0:
                j = np.where(toks == c)[0]
                assert len(j) == 1 and rw[seg][j[0]] == ws
            else:
                assert c not in toks


def _nearest_code_brute(q):
    vals = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    d = np.abs(q - vals)
    return int(np.argmin(d))  # argmin returns the first minimum = lowest code index


def test_fp4_qdq_closed_form(orc):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal(32 * 40) * np.repeat(np.exp2(rng.integers(-20, 20, 40)), 32))
    x = x.astype(np.float32)
    x[5] = 0.0
    x[40:72] = 0.0  # an all-zero block
    rc, out, sc, codes = orc.fp4_activation_qdq(x, 32)
    assert rc == 0
    for bi in range(40):
        blk = x[32 * bi:32 * bi + 32].astype(np.float64)
        amax = max(np.max(np.abs(blk)), 6 * 2.0 ** -126)
        scale = 2.0 ** (int(sc[bi]) - 127)
        # the smallest power of two that brings amax within 6
        assert amax / scale <= 6 and amax / (scale / 2) > 6
        for i in range(32):
            q = np.float32(np.clip(np.float32(blk[i]) / np.float32(scale), -6, 6))
            assert codes[32 * bi + i] == _nearest_code_brute(q)


# ---------------------------------------------------------------- vs the reference build

def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_synth_bf16_round_matches_ref(ref):
    """The product's own bf16 rounding of inputs (mvllm_hip.synth.bf16_round) equals the
    reference's bf16_round (src/quant/bf16.cpp:9-20) bit for bit over every high half with
    low halves that hit each rounding case: zero, just below / at / just above the tie,
    odd and even high halves (ties to even), subnormals, +-0, +-Inf, and NaNs whose
    payload lies in the low half only (truncated to +-Inf by the reference) or in both.
    Plus the reference's KATs (tests/test_host.cpp:8479-8483)."""
    from mvllm_hip import synth
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xC000, 0xFFFF], np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    x = bits.view(np.float32)
    got = synth.bf16_round(x).view(np.uint32)
    exp = ref.bf16_round_array(x).view(np.uint32)
    bad = np.nonzero(got != exp)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(exp[i])) for i in bad[:5]]
    assert synth.bf16_round(np.float32([1.00390625]))[0] == 1.0
    assert synth.bf16_round(np.float32([1.01171875]))[0] == 1.015625


def test_ref_scalars_bit_exact(orc, ref):
    rng = np.random.default_rng(21)
    vals = np.concatenate([rng.standard_normal(2000) * 10, [0.0, -0.0, 88.0, -88.0, 1e-30, 30.0,
                                                             -104.0, np.inf, -np.inf, np.nan]])
    vals = vals.astype(np.float32)
    for v in vals:
        v = float(v)
        for f, args in (("sigmoid", (v,)), ("clamped_swiglu", (v, v * 0.7, 7.0)),
                        ("clamped_swiglu", (v, -v, 0.0)), ("situ_glu", (v, v * 1.3, 4.0, 25.0)),
                        ("bf16_round", (v,))):
            a, b = orc.fn(f)(*args), ref.fn(f)(*args)
            assert _bits([a])[0] == _bits([b])[0] or (math.isnan(a) and math.isnan(b)), (f, v)
    for n in range(256):
        for f in ("mx4_scale", "e8m0_decode", "e2m1_decode"):
            a, b = orc.fn(f)(n), ref.fn(f)(n)
            assert _bits([a])[0] == _bits([b])[0] or (math.isnan(a) and math.isnan(b))
    for n in range(16):
        assert _bits([orc.fn("mx4_lut")(n)])[0] == _bits([ref.fn("mx4_lut")(n)])[0]


@pytest.mark.parametrize("fmt,S,K,O", [(0, 3, 64, 17), (4, 2, 256, 9), (4, 3, 100, 5),
                                       (7, 2, 224, 11), (7, 1, 45, 6), (8, 3, 200, 13),
                                       (8, 1, 7, 5)])
def test_ref_matmul_bit_exact(orc, ref, fmt, S, K, O):
    rng = np.random.default_rng(S * K + O)
    x = rng.standard_normal((S, K)).astype(np.float32)
    if fmt == 0:
        w, s = rng.standard_normal((O, K)).astype(np.float32), None
    elif fmt == 8:  # codes and scales from the reference's own quantize_int8_row
        wf = rng.standard_normal((O, K)).astype(np.float32)
        wf[0] = 0.0  # an all-zero row: scale 0, codes 0
        w, s = np.zeros((O, K), np.int8), np.zeros(O, np.float32)
        ref.lib.ref_quantize_int8_row(wf.ctypes.data, O, K, w.ctypes.data, s.ctypes.data)
        assert s[0] == 0 and not w[0].any() and np.abs(w).max() == 127
    elif fmt == 4:
        w = rng.integers(0, 256, size=(O, (K + 1) // 2), dtype=np.uint8)
        s = rng.uniform(0.005, 0.02, size=(O, (K + 63) // 64)).astype(np.float32)
    else:
        w = rng.integers(0, 256, size=(O, (K + 1) // 2), dtype=np.uint8)
        s = rng.integers(0, 256, size=(O, (K + 31) // 32), dtype=np.uint8)
    a, b = orc.matmul(fmt, x, w, s), ref.matmul(fmt, x, w, s)
    assert np.array_equal(_bits(a), _bits(b)) or np.array_equal(np.isnan(a), np.isnan(b))


@pytest.mark.parametrize("case", CASES)
def test_ref_moe_block_bit_exact(orc, ref, case):
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    rng = np.random.default_rng(D * 13 + I)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    o1, o2 = c.out.copy(), c.out.copy()
    assert orc.moe_block(*c.args(o1), act, a, b) == ref.moe_block(*c.args(o2), act, a, b) == 1
    assert np.array_equal(_bits(o1), _bits(o2))


def test_ref_topk_union_qdq_bit_exact(orc, ref):
    rng = np.random.default_rng(31)
    for _ in range(30):
        n = int(rng.integers(1, 30))
        k = int(rng.integers(1, n + 2))
        choice = rng.integers(-2, 3, size=n).astype(np.float32)
        mix = rng.uniform(-0.1, 1, size=n).astype(np.float32)
        r1, r2 = orc.moe_topk(choice, k, mix), ref.moe_topk(choice, k, mix)
        assert r1[0] == r2[0] and np.array_equal(r1[1], r2[1]) and \
            np.array_equal(_bits(r1[2]), _bits(r2[2]))
        idx = rng.integers(-1, 9, size=(5, 3)).astype(np.int32)
        assert np.array_equal(orc.moe_union_ids(idx, 5, 3, 6), ref.moe_union_ids(idx, 5, 3, 6))
    x = (rng.standard_normal(32 * 64) * np.repeat(np.exp2(rng.integers(-30, 30, 64)), 32))
    x = x.astype(np.float32)
    x[3], x[100], x[200] = np.nan, np.inf, -0.0
    for block in (32, 7):
        a, b = orc.fp4_activation_qdq(x, block), ref.fp4_activation_qdq(x, block)
        assert a[0] == b[0] == 0
        assert np.array_equal(a[2], b[2])
        assert np.array_equal(_bits(a[1]), _bits(b[1]))


# ---------------------------------------------------------------- native-FP4 composition

def _compose_fp4act_ref(lib, c, act, a, b):
    """The same composition built in Python from the reference build's own pieces
    (fp4_activation_qdq, matmul_mxfp4, the activation scalars) -- a second route to the
    numbers orc_moe_block_fp4act must produce bit for bit."""
    out = c.out.copy()
    actf = {0: lambda g, u: np.float32(lib.fn("sigmoid")(g)) * np.float32(g) * np.float32(u),
            1: lambda g, u: lib.fn("clamped_swiglu")(g, u, a),
            2: lambda g, u: lib.fn("situ_glu")(g, u, a, b)}[act]
    base = 0
    for e in range(c.nb):
        n = int(c.nr[e])
        if n <= 0:
            continue
        if c.g[e] is None:
            base += n
            continue
        xe = c.xg[int(c.xoff[e]):int(c.xoff[e]) + n]
        xq = np.stack([lib.fp4_activation_qdq(r, 32)[1] for r in xe])
        gt = lib.matmul(7, xq, c.g[e], c.gs[e])
        up = lib.matmul(7, xq, c.u[e], c.us[e])
        h = np.array([[actf(float(gv), float(uv)) for gv, uv in zip(gr, ur)]
                      for gr, ur in zip(gt, up)], np.float32)
        hq = np.stack([lib.fp4_activation_qdq(r, 32)[1] for r in h])
        y = lib.matmul(7, hq, c.d[e], c.ds[e])
        for r in range(n):
            dst = int(c.rows[base + r])
            if 0 <= dst < c.S:
                out[dst] = out[dst] + np.float32(c.rw[base + r]) * y[r]
        base += n
    return out


@pytest.mark.parametrize("act,a,b", [(2, 4.0, 25.0), (1, 7.0, 0.0)])
def test_fp4act_composition(orc, ref, act, a, b):
    """orc_moe_block_fp4act equals the composition of the reference build's own QDQ,
    MXFP4 GEMM and activation, bit for bit (silu_mul's product order is pinned by the
    moe_block tests; here the clamped and SiTU activations are composed)."""
    rng = np.random.default_rng(71 + act)
    c = random_case(rng, 7, 64, 96, [2, 0, 3, 1], 4, act, a, b, null_experts=(3,), invalid_rows=1)
    o1 = c.out.copy()
    assert orc.moe_block_fp4act(*c.args(o1), act, a, b) == 1
    o2 = _compose_fp4act_ref(ref, c, act, a, b)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))


def test_fp4act_close_to_f32(orc):
    """Quantizing activations to MXFP4 moves the block output by a bounded amount (the
    e2m1 grid is 1 part in 8 at worst), and fmt != 7 is refused."""
    rng = np.random.default_rng(72)
    c = random_case(rng, 7, 256, 128, [3, 2], 3, 2, 4.0, 25.0, zero_out=True)
    o1, o2 = c.out.copy(), c.out.copy()
    assert orc.moe_block_fp4act(*c.args(o1), 2, 4.0, 25.0) == 1
    assert orc.moe_block(*c.args(o2), 2, 4.0, 25.0) == 1
    err = npref.rel_err(o1, o2)
    assert 1e-4 < err < 0.3
    c4 = random_case(rng, 4, 64, 64, [1], 1)
    assert orc.moe_block_fp4act(*c4.args(), 0, 0.0, 0.0) == 0


# ---- the steps either side of the block: rmsnorm and the router ------------------------

def test_rmsnorm_bit_exact_vs_ref(orc, ref):
    """orc_rmsnorm equals quant::rmsnorm (src/quant/quant.cpp:384-398) bit for bit."""
    rng = np.random.default_rng(5)
    for n, eps, with_w in ((1, 1e-6, True), (7, 1e-5, False), (2048, 1e-6, True),
                           (7168, 1e-6, True), (333, 0.0, False)):
        x = (rng.standard_normal((3, n)) * rng.uniform(0.1, 50)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32) if with_w else None
        a, b = orc.rmsnorm(x, w, eps), ref.rmsnorm(x, w, eps)
        assert np.array_equal(_bits(a), _bits(b)), (n, eps, with_w)


def test_rmsnorm_closed_form(orc):
    """A row of equal values c normalises to sign(c) / sqrt(1 + eps / c^2) times w."""
    x = np.full((1, 64), -3.0, np.float32)
    w = np.full(64, 2.0, np.float32)
    y = orc.rmsnorm(x, w, 0.0)
    assert np.allclose(y, -2.0, rtol=1e-6, atol=0)


@pytest.mark.parametrize("D,E,k,rscale,ties", [(256, 64, 8, 1.0, False), (512, 384, 8, 2.5, False),
                                               (128, 32, 4, 1.0, True), (1024, 96, 6, 0.5, True)])
def test_norm_route_bit_exact_vs_ref(orc, ref, D, E, k, rscale, ties):
    """The oracle's rmsnorm -> cpu_route composition equals the reference's own router
    (file-local cpu_route, src/gpu/metal_ops.cpp:213-231, reached through its public host
    path metal_ops::layer_decode_full, :233-254): normalised row, picks and weights, bit for
    bit, with and without a bias, including equal router rows (ties: lower index first)."""
    rng = np.random.default_rng(D + E + k)
    w = (rng.standard_normal((E, D)) * 0.05).astype(np.float32)
    if ties:
        w[5] = w[2]
        w[E - 1] = w[0]
    post_ln = rng.uniform(0.5, 1.5, D).astype(np.float32)
    for rep in range(4):
        x = rng.standard_normal(D).astype(np.float32)
        bias = (rng.standard_normal(E) * 0.01).astype(np.float32) if rep % 2 else None
        nrm_r, idx_r, wt_r = ref.norm_route(x, post_ln, 1e-6, w, bias, k, rscale)
        nrm_o = orc.rmsnorm(x[None, :], post_ln, 1e-6)[0]
        idx_o, wt_o = orc.route(nrm_o, w, bias, k, rscale)
        assert np.array_equal(_bits(nrm_o), _bits(nrm_r))
        assert np.array_equal(idx_o[0], idx_r)
        assert np.array_equal(_bits(wt_o[0]), _bits(wt_r))


def test_route_closed_form(orc):
    """Identity router rows make each score exactly x[e]: the picks are the k largest
    sigmoid(x) + bias (ties to the lower index) and the weights their sigmoids over the
    sum, times rscale."""
    rng = np.random.default_rng(77)
    E = 48
    x = rng.permutation(np.linspace(-4, 4, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    w = np.eye(E, dtype=np.float32)
    idx, wt = orc.route(x, w, bias, 6, 1.5)
    sig = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    choice = sig + bias
    exp_idx = np.argsort(-choice, kind="stable")[:6]
    assert np.array_equal(idx[0], exp_idx)
    exp_w = sig[exp_idx] / sig[exp_idx].sum() * 1.5
    assert np.allclose(wt[0], exp_w, rtol=2e-6, atol=0)
