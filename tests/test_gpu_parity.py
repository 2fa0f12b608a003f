"""GPU parity: the HIP library (through its C ABI) against the CPU oracle.

Bars: dequantized weights, MXFP4 activation codes/scales and segment arrays are
bit-exact; the f32 GEMV path (decode) is within 2e-5 relative (max|y-ref| / max|ref|)
of the oracle, which itself equals the reference build bit for bit.
"""
import ctypes
import math
import sys

import numpy as np
import pytest
import torch

import npref
from cases import random_case

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_lists(c):
    keep = []

    def L(xs):
        if xs is None:
            return None
        out = []
        for x in xs:
            t = dev(x)
            keep.append(t)
            out.append(None if t is None else t.data_ptr())
        return out
    return [L(c.g), L(c.u), L(c.d), L(c.gs), L(c.us), L(c.ds)], keep


def run_dev(hip, c, act, a, b, stream=None):
    lists, keep = dev_lists(c)
    xg = dev(c.xg)
    out = dev(c.out)
    hip.moe_block_dev(c.nb, c.D, c.I, c.fmt, *lists, xg, c.xoff, c.nr, c.rows, c.rw, out, c.S,
                      act, a, b, stream=stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_out(orc, c, act, a, b):
    o = c.out.copy()
    assert orc.moe_block(*c.args(o), act, a, b) == 1
    return o


# ------------------------------------------------------------- bit-exact formats

@pytest.mark.parametrize("fmt,O,K,offset", [(4, 64, 2048, 0), (4, 33, 1024, 0), (4, 9, 96, 0),
                                            (4, 5, 77, 0), (4, 8, 256, 3), (7, 64, 7168, 0),
                                            (7, 17, 2048, 0), (7, 6, 45, 0), (7, 8, 256, 1)])
def test_dequant_bit_exact(hip, orc, fmt, O, K, offset):
    say("dequant", fmt, O, K, offset)
    rng = np.random.default_rng(O * K + fmt)
    packed = rng.integers(0, 256, size=(O, (K + 1) // 2), dtype=np.uint8)
    if fmt == 4:
        scales = rng.uniform(-0.03, 0.03, size=(O, (K + 63) // 64)).astype(np.float32)
        scales.flat[::7] = 0.0
    else:
        scales = rng.integers(0, 256, size=(O, (K + 31) // 32), dtype=np.uint8)
    # offset > 0 misaligns the packed base and forces the element-wise path
    pbuf = torch.zeros(packed.size + 16, dtype=torch.uint8, device="cuda")
    pbuf[offset:offset + packed.size] = torch.from_numpy(packed.ravel()).cuda()
    s_d = dev(scales)
    w = torch.empty((O, K), dtype=torch.float32, device="cuda")
    hip.dequant(fmt, pbuf[offset:], s_d, O, K, w)
    got = w.cpu().numpy()
    exp = orc.dequant(fmt, packed, scales, O, K)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    m = ~np.isnan(exp)
    assert np.array_equal(got[m].view(np.uint32), exp[m].view(np.uint32))


@pytest.mark.parametrize("fmt,O,K", [(4, 48, 2048), (4, 16, 1024), (7, 48, 7168), (7, 16, 1024)])
def test_dequant_bit_exact_mfma_decode(hip, orc, fmt, O, K):
    """The weights exactly as the matrix-core path decodes them (bf16 operands), checked
    bit for bit, including zero/infinite ue8m0 scale bytes."""
    say("dequant mfma path", fmt, O, K)
    rng = np.random.default_rng(O + K + 7 * fmt)
    packed = rng.integers(0, 256, size=(O, K // 2), dtype=np.uint8)
    if fmt == 4:
        scales = rng.uniform(-0.03, 0.03, size=(O, K // 64)).astype(np.float32)
    else:
        scales = rng.integers(1, 255, size=(O, K // 32), dtype=np.uint8)
        scales[0, :4] = [0, 255, 1, 254]
    w = torch.empty((O, K), dtype=torch.float32, device="cuda")
    assert hip.set_option("dequant_path", 1)
    try:
        hip.dequant(fmt, dev(packed), dev(scales), O, K, w)
    finally:
        hip.set_option("dequant_path", 0)
    got = w.cpu().numpy()
    exp = orc.dequant(fmt, packed, scales, O, K)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    m = ~np.isnan(exp)
    bad = np.argwhere(got[m].view(np.uint32) != exp[m].view(np.uint32))
    assert bad.size == 0, (got[m][bad[:5, 0]], exp[m][bad[:5, 0]])


def test_quantize_mxfp4_bit_exact(hip, orc):
    say("quantize_mxfp4")
    rng = np.random.default_rng(77)
    n, K = 12, 512
    x = rng.standard_normal((n, K)) * np.repeat(np.exp2(rng.integers(-40, 40, (n, K // 32))),
                                                 32, axis=1)
    x = x.astype(np.float32)
    x[0, :32] = 0.0
    x[1, 5], x[2, 7], x[3, 9] = np.nan, np.inf, -np.inf
    x[4, :32] = np.float32(0.25) * (np.arange(32) % 13)  # exact ties between codes
    x[5, :32] = np.float32(2.0 ** -130) * (np.arange(32) % 7)  # scale 2^-127, subnormals
    codes = torch.zeros((n, K // 2), dtype=torch.uint8, device="cuda")
    scales = torch.zeros((n, K // 32), dtype=torch.uint8, device="cuda")
    planes = torch.full((n, K), -1, dtype=torch.int16, device="cuda")
    hip.quantize_mxfp4(dev(x), n, K, codes, scales, planes)
    cg, sg = codes.cpu().numpy(), scales.cpu().numpy()
    pg = planes.cpu().numpy().view(np.uint16)
    for r in range(n):
        rc, q, sc, cd = orc.fp4_activation_qdq(x[r], 32)
        assert np.array_equal(sg[r], sc), r
        assert np.array_equal(npref.unpack_nibbles(cg[r:r + 1], K)[0], cd), r
        # the bf16 copy of the reference's QDQ output: exact (its low half is zero)
        qb = q.view(np.uint32)
        assert np.all((qb & 0xffff) == 0), r
        assert np.array_equal(pg[r], (qb >> 16).astype(np.uint16)), r


@pytest.mark.parametrize("fmt", [4, 7])
def test_bf16_planes_bit_exact(hip, fmt):
    """The device's bf16 activation terms against the reference's bf16_round
    (src/quant/bf16.cpp:9-20), through mvllm_hip.synth.bf16_round, which the CPU suite pins
    to the reference build bit for bit.  The same conversion (split_terms) feeds the
    grouped GEMM's planes, the decode kernels' activations and H.  Every term count:
    plane 0 = bf16_round(x), plane 1 = bf16_round(x - plane 0) (0 for non-finite plane 0),
    plane 2 = bf16_round of the next remainder.  Values: random magnitudes over the whole
    exponent range, exact ties (even and odd), subnormals, +-0, +-Inf and quiet NaN.  A NaN
    whose payload lies only in the low 16 bits is left out: the reference truncates it to
    Inf, the device's converter keeps it a NaN (no bf16_round'ed input is such a NaN)."""
    from mvllm_hip import synth
    say("bf16 planes", fmt)
    rng = np.random.default_rng(41 + fmt)
    n, K = 8, 512
    hi = rng.integers(0, 1 << 16, size=n * K, dtype=np.uint32)
    lo = rng.choice(np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32), size=n * K)
    bits = (hi << 16) | lo
    bits[:8] = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00008000,
                0x00018000, 0x807F8000]
    expo_all_ones = (bits & 0x7F800000) == 0x7F800000
    low_only_nan = expo_all_ones & ((bits & 0x007F0000) == 0) & ((bits & 0xFFFF) != 0)
    bits[low_only_nan] = 0x7FC00000
    x = bits.view(np.float32).reshape(n, K)
    # element e of an 8-block is stored at a_slot(e): int4 order 0 2 4 6 1 3 5 7
    slot = np.array([0, 4, 1, 5, 2, 6, 3, 7]) if fmt == 4 else np.arange(8)
    for terms in (1, 2, 3):
        planes = torch.zeros((terms, n, K), dtype=torch.int16, device="cuda")
        hip.bf16_planes(fmt, terms, dev(x), n, K, planes)
        got = planes.cpu().numpy().view(np.uint16).reshape(terms, n, K // 8, 8)
        got = got[..., slot].reshape(terms, n, K)
        rem = x.copy()
        for tm in range(terms):
            exp = synth.bf16_round(rem)
            eb = (exp.view(np.uint32) >> 16).astype(np.uint16)
            nan = np.isnan(exp)
            got_nan = ((got[tm] & 0x7F80) == 0x7F80) & ((got[tm] & 0x7F) != 0)
            assert np.array_equal(got_nan, nan), (terms, tm)
            ok = got[tm][~nan] == eb[~nan]
            assert ok.all(), (terms, tm, np.nonzero(~ok)[0][:5])
            with np.errstate(invalid="ignore"):
                nxt = (rem - exp).astype(np.float32)
            rem = np.where(np.isfinite(exp), nxt, np.float32(0)).astype(np.float32)


# ------------------------------------------------------------- f32 GEMV parity

DEV_CASES = [
    # fmt, D, I, nr, S, act, a, b, null_experts, invalid_rows
    (4, 1024, 512, [1, 1], 1, 1, 7.0, 0.0, (), 0),                 # c0 shape
    (4, 2048, 1024, [1] * 8, 1, 0, 0.0, 0.0, (), 0),               # c1 T=1 shape
    (4, 2048, 1024, [2, 3, 1, 4, 2], 4, 0, 0.0, 0.0, (), 0),       # NR 4
    (4, 512, 256, [8, 5, 16, 1], 16, 1, 7.0, 0.0, (), 0),          # NR 8 and > 8 rows
    (4, 256, 128, [1, 2, 0, 3], 4, 1, 7.0, 0.0, (1,), 2),          # skips + invalid rows
    (4, 96, 70, [2, 1], 3, 1, 0.0, 0.0, (), 0),                    # odd I: generic down
    (4, 77, 33, [1, 2], 2, 0, 0.0, 0.0, (), 0),                    # odd everything
    (7, 7168, 2048, [1, 1, 1], 1, 2, 4.0, 25.0, (), 0),            # c2 shape
    (7, 1024, 512, [3, 1, 2, 6], 6, 2, 4.0, 25.0, (), 1),
    (7, 65, 31, [1, 1], 2, 2, 4.0, 25.0, (), 0),
    (0, 64, 48, [2, 1], 3, 1, 3.0, 0.0, (0,), 0),                  # f32 weights
    (4, 2048, 1024, [7, 1, 13], 16, 1, 7.0, 0.0, (), 0),           # rows > one item
    (7, 2048, 1024, [5, 9], 12, 2, 4.0, 25.0, (), 0),
]


@pytest.mark.parametrize("case", [DEV_CASES[1], DEV_CASES[7], DEV_CASES[-2]])
def test_moe_block_bf16_mode(hip, orc, case):
    """mode 2: activations rounded to bf16 (one term) -- the north-star tolerance 1e-2."""
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("bf16 mode", case)
    rng = np.random.default_rng(D * 3 + I)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    assert hip.set_option("mode", 2)
    try:
        got = run_dev(hip, c, act, a, b)
    finally:
        hip.set_option("mode", 0)
    exp = oracle_out(orc, c, act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < 1e-2


@pytest.mark.parametrize("case", DEV_CASES)
def test_moe_block_dev_parity(hip, orc, case):
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("moe_block_dev", case)
    rng = np.random.default_rng(D * 31 + I + len(nr))
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    got = run_dev(hip, c, act, a, b)
    exp = oracle_out(orc, c, act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < TOL_F32


@pytest.mark.parametrize("ci,ks", [(1, 1), (1, 2), (1, 4), (7, 2), (7, 4), (-2, 1), (-2, 2),
                                   (-2, 4)])
def test_decode_k_split_parity(hip, orc, ci, ks):
    """Every K split of the decode kernels that both projections admit (option dec_ks),
    including those the planner does not pick for these shapes."""
    fmt, D, I, nr, S, act, a, b, nulls, bad = case = DEV_CASES[ci]
    say("dec_ks", ks, case)
    rng = np.random.default_rng(D * 41 + I + ks)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    hip.stats_reset()
    assert hip.set_option("dec_ks", ks)
    try:
        got = run_dev(hip, c, act, a, b)
    finally:
        hip.set_option("dec_ks", 0)
    exp = oracle_out(orc, c, act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err, hip.stats())
    assert err < TOL_F32


@pytest.mark.parametrize("inline", [0, 1])
@pytest.mark.parametrize("ci", [1, 3, 7, "many"])
def test_decode_descriptor_paths(hip, orc, ci, inline):
    """Gate/up descriptors in the kernel arguments (dec_inline 1, default) or read from
    the pinned plan slot (0); 'many' has 70 items, past the 64 the arguments carry, so
    it takes the slot either way."""
    case = (4, 512, 256, [1] * 70, 16, 1, 7.0, 0.0, (), 0) if ci == "many" else DEV_CASES[ci]
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("dec_inline", inline, ci)
    rng = np.random.default_rng(D * 43 + I + inline)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    assert hip.set_option("dec_inline", inline)
    try:
        got = run_dev(hip, c, act, a, b)
    finally:
        hip.set_option("dec_inline", 1)
    exp = oracle_out(orc, c, act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < TOL_F32


@pytest.mark.parametrize("case", DEV_CASES[::2])
def test_moe_block_host_parity(hip, orc, case):
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("moe_block host", case)
    rng = np.random.default_rng(D * 37 + I)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    got = c.out.copy()
    assert hip.moe_block(*c.args(got), act, a, b) == 1
    exp = oracle_out(orc, c, act, a, b)
    assert npref.rel_err(got, exp) < TOL_F32
    # rows that receive nothing are untouched bit for bit
    touched = set(int(r) for r in c.rows if 0 <= r < c.S)
    for t in range(c.out.shape[0]):
        if t not in touched:
            assert np.array_equal(got[t], c.out[t])


def test_validation_matches_reference(hip):
    say("validation")
    rng = np.random.default_rng(5)
    c = random_case(rng, 4, 64, 64, [1], 1)
    for k, v in ((0, 0), (1, 0), (3, 5), (10, None), (11, None), (12, None), (15, None)):
        args = list(c.args())
        args[k] = v
        assert hip.moe_block(*args, 0, 0.0, 0.0, check=False) == 0
    args = list(c.args())
    args[13] = None  # rows == NULL: nothing reaches out
    o = args[15]
    assert hip.moe_block(*args, 0, 0.0, 0.0) == 1 and np.array_equal(o, c.out)


@pytest.mark.parametrize("D,I", [(256, 128), (512, 512)])
def test_nonfinite_propagation(hip, orc, D, I):
    """Inf scales / activations: NaN and Inf land where the reference puts them, on the
    element-wise path (256 x 128) and through the matrix-core decode kernels (512 x 512:
    chains over n - 8, exact redo of tiles with out-of-range scales)."""
    say("nonfinite", D, I)
    rng = np.random.default_rng(8)
    for fmt in (4, 7):
        c = random_case(rng, fmt, D, I, [1, 1, 1], 3, 2 if fmt == 7 else 1, 4.0, 25.0)
        c.rows[:] = [0, 1, 2]
        if fmt == 7:
            c.gs[0][5, 2] = 255      # +inf scale in one gate group of expert 0
            c.ds[1][7, 1] = 0        # zero scale in one down group of expert 1
        else:
            c.gs[0][5, 1] = np.inf
            c.ds[1][7, 0] = -np.inf
        c.xg[2, 17] = np.inf
        got = run_dev(hip, c, c.act, c.a, c.b)
        exp = oracle_out(orc, c, c.act, c.a, c.b)
        assert np.array_equal(np.isnan(got), np.isnan(exp))
        assert np.array_equal(np.isinf(got), np.isinf(exp))
        fin = np.isfinite(exp)
        assert np.array_equal(np.sign(got[np.isinf(exp)]), np.sign(exp[np.isinf(exp)]))
        assert npref.rel_err(got[fin], exp[fin]) < TOL_F32


@pytest.mark.parametrize("fmt", [4, 7])
@pytest.mark.parametrize("path,D,I,gemm", [("elementwise", 256, 128, 0), ("decode", 512, 512, 2),
                                           ("gemm", 512, 256, 1)])
def test_clamp_swiglu_nonfinite_up(hip, orc, fmt, path, D, I, gemm):
    """ClampSwiGLU with a non-finite up projection: the reference clamps `up` with
    comparisons (src/quant/quant.hpp:37-50), so a NaN up stays NaN and reaches the row's
    down outputs; an infinite one is clamped to +-limit.  The up scales alone carry the
    non-finite values (MXFP4 byte 255 on a zero nibble gives 0 * inf = NaN; an int4 scale
    of inf or NaN), on the element-wise, decode and grouped-GEMM paths."""
    say("clamp nonfinite up", fmt, path)
    rng = np.random.default_rng(19 + fmt + D)
    c = random_case(rng, fmt, D, I, [2, 1, 3], 6, 1, 7.0, 0.0)
    c.rows[:] = np.arange(6, dtype=np.int32)
    if fmt == 7:
        c.us[0][3, 1] = 255            # +inf block scale: NaN where the nibble is +-0
        c.us[2][5, 0] = 255
    else:
        c.us[0][3, 1] = np.nan
        c.us[2][5, 0] = np.inf
    assert hip.set_option("gemm", gemm)
    try:
        got = run_dev(hip, c, 1, 7.0, 0.0)
    finally:
        hip.set_option("gemm", 0)
    exp = oracle_out(orc, c, 1, 7.0, 0.0)
    assert np.isnan(exp).any()  # the case reaches the clamp with a NaN up
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    fin = np.isfinite(exp)
    tol = TOL_F32 if gemm != 1 else 1e-2
    assert npref.rel_err(got[fin], exp[fin]) < tol


# ------------------------------------------------------------- benchmark configs

@pytest.mark.parametrize("name,T", [("c0", 1), ("c1", 1), ("c1", 4), ("c1", 16), ("c2", 1)])
def test_config_parity(hip, orc, name, T):
    from mvllm_hip import synth
    say("config", name, T)
    w = synth.make_workload(name, T=T)
    g, u, d, gs, us, ds = w.lists()
    out = np.zeros((T, w.D), np.float32)
    exp = out.copy()
    assert orc.moe_block(w.nb, w.D, w.I, w.fmt, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows,
                         w.rw, exp, T, w.act, w.a, w.b) == 1
    from cases import Case
    c = Case(w.nb, w.D, w.I, w.fmt, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, out,
             T, w.act, w.a, w.b)
    got = run_dev(hip, c, w.act, w.a, w.b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < TOL_F32
    # the drop-in host entry gives the same result
    got2 = out.copy()
    hip.moe_block(w.nb, w.D, w.I, w.fmt, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw,
                  got2, T, w.act, w.a, w.b)
    assert npref.rel_err(got2, exp) < TOL_F32


# ------------------------------------------------------------- residency / staging

@pytest.mark.parametrize("n_experts", [300, 600])
def test_tier_table_entries(hip, n_experts):
    """mvllm_hip_tier_table writes each expert's HBM copy address (resident_ptr) or null,
    for tables in a kernel's arguments (<= 448 entries) and through the pinned ring
    (larger), the ring wrapped around more than once."""
    L = hip.lib()
    nbytes = 4096
    layer = 40 + n_experts  # a layer no other test uses
    eids = [0, 7, n_experts // 2 + 1, n_experts - 1]
    blobs = []
    for i, e in enumerate(eids):
        p = L.mvllm_hip_host_alloc(nbytes)
        assert p
        ctypes.memset(p, i + 1, nbytes)
        blobs.append(p)
        hip.promote(p, nbytes, layer, e)
    torch.cuda.synchronize()
    try:
        want = np.zeros(n_experts, np.uint64)
        for e in eids:
            want[e] = L.mvllm_hip_resident_ptr(layer, e)
            assert want[e]
        tab = torch.full((n_experts,), -1, dtype=torch.int64, device="cuda")
        for rep in range(11):  # more calls than the ring has slots
            tab.fill_(-1)
            assert hip.tier_table(layer, n_experts, tab) == len(eids)
            hip.tier_table_done(layer)
            got = tab.cpu().numpy().view(np.uint64)
            assert np.array_equal(got, want), rep
    finally:
        for e in eids:
            hip.evict(layer, e)
        torch.cuda.synchronize()
        for p in blobs:
            L.mvllm_hip_host_free(p)


def test_promote_hits_and_evict(hip, orc):
    from mvllm_hip import synth
    say("promote")
    w = synth.make_workload("c0", T=1)
    n, off = hip.expert_geom(4, w.D, w.I)
    blobs = []
    L = hip.lib()
    for e in w.eids:
        p = L.mvllm_hip_host_alloc(n)
        assert p
        buf = (ctypes.c_uint8 * n).from_address(p)
        arr = np.frombuffer(buf, np.uint8)
        ex = w.experts[int(e)]
        for piece, o in zip(("gp", "gs", "up", "us", "dp", "ds"), off):
            b = ex[piece].view(np.uint8).ravel()
            arr[o:o + b.size] = b
        blobs.append((p, arr))
    views = []
    for p, arr in blobs:
        v = {}
        for piece, o in zip(("gp", "gs", "up", "us", "dp", "ds"), off):
            src = w.experts[int(w.eids[0])][piece]
            v[piece] = np.frombuffer((ctypes.c_uint8 * (src.nbytes)).from_address(p + int(o)),
                                     src.dtype).reshape(src.shape)
        views.append(v)
    g = [v["gp"] for v in views]
    u = [v["up"] for v in views]
    d = [v["dp"] for v in views]
    gs = [v["gs"] for v in views]
    us = [v["us"] for v in views]
    ds = [v["ds"] for v in views]
    exp = np.zeros((1, w.D), np.float32)
    orc.moe_block(w.nb, w.D, w.I, 4, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, exp,
                  1, w.act, w.a, w.b)
    hip.stats_reset()
    # 1) nothing resident: misses, copied in
    o1 = np.zeros((1, w.D), np.float32)
    hip.moe_block(w.nb, w.D, w.I, 4, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, o1,
                  1, w.act, w.a, w.b)
    st = hip.stats()
    assert st["misses"] == w.nb and st["resident_hits"] == 0
    # 2) promote both: hits
    for i, (p, arr) in enumerate(blobs):
        hip.promote(p, n, 0, int(w.eids[i]))
    o2 = np.zeros((1, w.D), np.float32)
    hip.moe_block(w.nb, w.D, w.I, 4, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, o2,
                  1, w.act, w.a, w.b)
    st = hip.stats()
    assert st["resident_hits"] == w.nb and st["promotions"] == w.nb
    assert npref.rel_err(o1, exp) < TOL_F32 and npref.rel_err(o2, exp) < TOL_F32
    # 3) evict one: one hit, one miss; the slot's new content is picked up
    assert hip.evict(0, int(w.eids[0]))
    blobs[0][1][:] = blobs[1][1][:]  # the store reused slot 0 for expert eids[1]
    o3 = np.zeros((1, w.D), np.float32)
    hip.moe_block(w.nb, w.D, w.I, 4, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, o3,
                  1, w.act, w.a, w.b)
    g2, u2, d2 = [g[1], g[1]], [u[1], u[1]], [d[1], d[1]]
    gs2, us2, ds2 = [gs[1], gs[1]], [us[1], us[1]], [ds[1], ds[1]]
    exp3 = np.zeros((1, w.D), np.float32)
    orc.moe_block(w.nb, w.D, w.I, 4, g2, u2, d2, gs2, us2, ds2, w.xg, w.xoff, w.nr, w.rows, w.rw,
                  exp3, 1, w.act, w.a, w.b)
    assert npref.rel_err(o3, exp3) < TOL_F32
    for p, _ in blobs:
        L.mvllm_hip_host_free(p)
    for e in w.eids:
        hip.evict(0, int(e))


def test_two_streams_in_sequence(hip, orc):
    say("two streams")
    rng = np.random.default_rng(44)
    c1 = random_case(rng, 4, 1024, 512, [2, 1, 3], 4, 1, 7.0, 0.0)
    c2 = random_case(rng, 7, 1024, 512, [1, 2], 4, 2, 4.0, 25.0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    l1, k1 = dev_lists(c1)
    l2, k2 = dev_lists(c2)
    x1, o1 = dev(c1.xg), dev(c1.out)
    x2, o2 = dev(c2.xg), dev(c2.out)
    torch.cuda.synchronize()
    hip.moe_block_dev(c1.nb, c1.D, c1.I, 4, *l1, x1, c1.xoff, c1.nr, c1.rows, c1.rw, o1, c1.S,
                      1, 7.0, 0.0, stream=s1)
    hip.moe_block_dev(c2.nb, c2.D, c2.I, 7, *l2, x2, c2.xoff, c2.nr, c2.rows, c2.rw, o2, c2.S,
                      2, 4.0, 25.0, stream=s2)
    torch.cuda.synchronize()
    assert npref.rel_err(o1.cpu().numpy(), oracle_out(orc, c1, 1, 7.0, 0.0)) < TOL_F32
    assert npref.rel_err(o2.cpu().numpy(), oracle_out(orc, c2, 2, 4.0, 25.0)) < TOL_F32


# ------------------------------------------------------------- grouped GEMM (prefill)

TOL_BF16 = 1e-2   # one bf16 term per activation (the prefill arithmetic)
TOL_2TERM = 5e-5  # two bf16 terms per activation (mode 1)

GEMM_CASES = [
    # fmt, D, I, nr, S, act, a, b, null_experts, invalid_rows
    (4, 1024, 512, [40, 17, 3, 70, 1], 64, 1, 7.0, 0.0, (), 0),   # row classes 1/2, 2-3 blocks
    (4, 256, 256, [16, 33], 40, 0, 0.0, 0.0, (), 0),              # one K step
    (4, 512, 256, [20, 5, 9], 30, 1, 7.0, 0.0, (1,), 3),          # skips + invalid rows
    (7, 1024, 512, [200, 5, 33, 64, 129], 256, 2, 4.0, 25.0, (), 0),  # classes 1/2/4/8
    (7, 512, 768, [18, 140], 160, 2, 4.0, 25.0, (0,), 2),
    (7, 256, 256, [1, 2, 3], 6, 0, 0.0, 0.0, (), 0),
]


def _gemm_run(hip, c, mode, gemm=1):
    assert hip.set_option("gemm", gemm) and hip.set_option("mode", mode)
    try:
        return run_dev(hip, c, c.act, c.a, c.b)
    finally:
        hip.set_option("gemm", 0)
        hip.set_option("mode", 0)


@pytest.mark.parametrize("case", GEMM_CASES)
@pytest.mark.parametrize("mode,tol", [(0, TOL_BF16), (1, TOL_2TERM)])
def test_gemm_parity(hip, case, mode, tol):
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("gemm", mode, case)
    rng = np.random.default_rng(D * 17 + I + sum(nr))
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    got = _gemm_run(hip, c, mode)
    exp = npref.moe_block64(*c.args(), act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < tol
    # rows that receive nothing are untouched
    touched = set(int(r) for r in c.rows if 0 <= r < c.S)
    for t in range(c.out.shape[0]):
        if t not in touched:
            assert np.array_equal(got[t], c.out[t])


@pytest.mark.parametrize("case", [GEMM_CASES[0], GEMM_CASES[3], GEMM_CASES[4]])
def test_gemm_task_order(hip, case):
    """Option gemm_xcd only reorders the tasks over the XCDs: every output element comes
    from the same tile and the same summation, so results are bit-identical."""
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("gemm task order", case)
    rng = np.random.default_rng(D * 17 + I + sum(nr))
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    base = _gemm_run(hip, c, 0)
    assert hip.set_option("gemm_xcd", 0)
    try:
        other = _gemm_run(hip, c, 0)
    finally:
        hip.set_option("gemm_xcd", 1)
    assert np.array_equal(base.view(np.uint32), other.view(np.uint32))


@pytest.mark.parametrize("fmt,D,I,nr,act,a,b", [
    (4, 6144, 2048, [40, 21, 1], 1, 7.0, 0.0),          # c3 shapes
    (7, 7168, 2048, [130, 3, 17], 2, 4.0, 25.0),         # c4 shapes, a full 128-row block
])
def test_gemm_real_shapes(hip, fmt, D, I, nr, act, a, b):
    """Full-size prefill expert shapes; the grouped GEMM is picked automatically
    (some expert has more than 16 rows)."""
    say("gemm real", fmt, D, I, nr)
    rng = np.random.default_rng(D + I + fmt)
    c = random_case(rng, fmt, D, I, nr, 64, act, a, b)
    got = run_dev(hip, c, act, a, b)
    exp = npref.moe_block64(*c.args(), act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < TOL_BF16


@pytest.mark.parametrize("fmt", [4, 7])
def test_gemm_nonfinite(hip, orc, fmt):
    """Nonfinite and out-of-range scales through the grouped GEMM (row classes 1 to 8 for
    MXFP4): scale bytes 0, 1 and 255 send their task through the exact redo, and NaN and
    Inf land where the reference puts them."""
    say("gemm nonfinite", fmt)
    rng = np.random.default_rng(81 + fmt)
    nr = [20, 40, 3, 100] if fmt == 7 else [20, 3, 30]
    c = random_case(rng, fmt, 512, 256, nr, 48, 2 if fmt == 7 else 1, 4.0, 25.0)
    if fmt == 7:
        c.gs[0][5, 2] = 255      # +inf scale in one gate group of expert 0
        c.ds[1][7, 1] = 0        # zero scale in one down group of expert 1
        c.us[2][3, 0] = 1        # subnormal products in one up group of expert 2
        c.gs[3][9, 4] = 254      # products up to 6 * 2^127 in one gate group of expert 3
    else:
        c.gs[0][5, 1] = np.inf
        c.ds[1][7, 0] = -np.inf
    c.xg[25, 17] = np.inf
    got = _gemm_run(hip, c, 0)
    exp = oracle_out(orc, c, c.act, c.a, c.b)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    assert np.array_equal(np.sign(got[np.isinf(exp)]), np.sign(exp[np.isinf(exp)]))
    fin = np.isfinite(exp)
    assert npref.rel_err(got[fin], exp[fin]) < TOL_BF16


@pytest.mark.parametrize("name,T", [("c3", 16), ("c4", 8)])
def test_prefill_config_parity(hip, orc, name, T):
    """Prefill configurations at a token count the oracle finishes in seconds, through the
    grouped GEMM, against the reference restatement."""
    from mvllm_hip import synth
    from cases import Case
    say("prefill config", name, T)
    w = synth.make_workload(name, T=T)
    g, u, d, gs, us, ds = w.lists()
    out = np.zeros((T, w.D), np.float32)
    exp = out.copy()
    assert orc.moe_block(w.nb, w.D, w.I, w.fmt, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows,
                         w.rw, exp, T, w.act, w.a, w.b) == 1
    c = Case(w.nb, w.D, w.I, w.fmt, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, out,
             T, w.act, w.a, w.b)
    for mode, tol in ((0, TOL_BF16), (1, TOL_2TERM)):
        got = _gemm_run(hip, c, mode)
        err = npref.rel_err(got, exp)
        say("  mode", mode, "rel_err", err)
        assert err < tol


# ------------------------------------------------------------- native MXFP4 activations

FP4_CASES = [
    # D, I, nr, S, act, a, b
    (1024, 512, [20, 5, 70, 1], 64, 2, 4.0, 25.0),    # bf16 classes 1/2, FP4 class 8
    # an expert of three blocks (two 256-row FP4 items run column block by column block,
    # then an 88-row one), a 64-row-class expert, the bf16 classes
    (1024, 512, [600, 40, 20, 5], 160, 2, 4.0, 25.0),
    # K / 256 odd in the down projection (768 = 3 x 256): a row's 24 scale bytes end
    # inside a 16-byte scale load, the last row's at the end of the buffer
    (512, 768, [40, 90, 200], 96, 1, 7.0, 0.0),
    (7168, 2048, [3, 40], 16, 2, 4.0, 25.0),           # K3 shapes
    (512, 256, [1, 1, 2], 3, 1, 7.0, 0.0),             # decode-shaped, clamped SwiGLU
]


def _fp4_run(hip, c):
    assert hip.set_option("fp4act", 1)
    try:
        return run_dev(hip, c, c.act, c.a, c.b)
    finally:
        hip.set_option("fp4act", 0)


def _fp4_check(got, exp):
    """Products of e2m1 values are exact, so the path differs from the composed oracle by
    summation order -- except where that order moves an h value across an e2m1 rounding
    boundary before the down projection (rare; one code step of one h element)."""
    den = np.max(np.abs(exp))
    dev_ = np.abs(got.astype(np.float64) - exp) / den
    say("  rel_err max", float(dev_.max()), "p99", float(np.quantile(dev_, 0.99)))
    assert float(dev_.max()) < 1e-2
    assert float(np.quantile(dev_, 0.99)) < 1e-5


@pytest.mark.parametrize("case", FP4_CASES)
def test_fp4act_parity(hip, orc, case):
    D, I, nr, S, act, a, b = case
    say("fp4act", case)
    rng = np.random.default_rng(D + 3 * I + len(nr))
    c = random_case(rng, 7, D, I, nr, S, act, a, b)
    got = _fp4_run(hip, c)
    exp = c.out.copy()
    assert orc.moe_block_fp4act(*c.args(exp), act, a, b) == 1
    _fp4_check(got, exp)


def test_fp4act_config_c4(hip, orc):
    """Config c4 (K3 MXFP4, Zipf routing) at T=8 against the composed oracle; the same
    call with f32 activations stays within the quantization distance of the reference."""
    from mvllm_hip import synth
    from cases import Case
    say("fp4act c4 T=8")
    w = synth.make_workload("c4", T=8)
    g, u, d, gs, us, ds = w.lists()
    out = np.zeros((8, w.D), np.float32)
    c = Case(w.nb, w.D, w.I, w.fmt, g, u, d, gs, us, ds, w.xg, w.xoff, w.nr, w.rows, w.rw, out,
             8, w.act, w.a, w.b)
    got = _fp4_run(hip, c)
    exp = out.copy()
    assert orc.moe_block_fp4act(*c.args(exp), w.act, w.a, w.b) == 1
    _fp4_check(got, exp)


@pytest.mark.parametrize("act,a,b", [(2, 4.0, 25.0), (1, 7.0, 0.0)])
def test_fp4act_special_scale_bytes(hip, orc, act, a, b):
    """Weight scale bytes 0, 1, 254 and 255 in gate, up and down under fp4act, in every
    row class (bf16 16/32-row classes; scaled-FP4 64-, 128- and 256-row blocks).  The
    matrix cores read byte 0 as 2^-127 and 255 as NaN where the reference's mx4_scale gives
    +0 and +inf (src/quant/quant.hpp:12-20): NaN and +-inf must land where the composed
    oracle puts them, and the finite part must meet the fp4act bar."""
    say("fp4act special scale bytes", act)
    rng = np.random.default_rng(4242 + act)
    # 70 rows: 128-row FP4 class; 40: 64-row; 300: a 256-row block + a 44-row one;
    # 20: bf16 32-row class; 130: 256-row class
    nr = [70, 40, 300, 20, 130]
    c = random_case(rng, 7, 512, 256, nr, 600, act, a, b)
    c.gs[0][5, 2] = 255
    c.us[0][9, 3] = 0
    c.ds[1][7, 1] = 255
    c.ds[1][100, 0] = 0
    c.gs[2][200, 15] = 255   # the last byte of its row
    c.us[2][3, 0] = 1
    c.ds[2][511, 7] = 255    # the last byte of the buffer
    c.gs[3][9, 4] = 254
    c.ds[3][3, 3] = 255
    c.ds[4][50, 2] = 0
    c.gs[4][77, 6] = 1
    c.us[4][30, 1] = 255
    got = _fp4_run(hip, c)
    exp = c.out.copy()
    assert orc.moe_block_fp4act(*c.args(exp), act, a, b) == 1
    n_nan, n_inf = int(np.isnan(exp).sum()), int(np.isinf(exp).sum())
    say("  oracle: nan", n_nan, "inf", n_inf)
    assert n_nan + n_inf > 0
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    assert np.array_equal(np.sign(got[np.isinf(exp)]), np.sign(exp[np.isinf(exp)]))
    fin = np.isfinite(exp)
    _fp4_check(got[fin], exp[fin])


@pytest.mark.parametrize("case", [DEV_CASES[1], DEV_CASES[3], DEV_CASES[7], DEV_CASES[-2]])
def test_combine_ordered_vs_atomic(hip, orc, case):
    """Decode calls fold the combine into the down kernel (float atomics, any order);
    option combine_ordered runs the separate combine in the reference's order.  Both meet
    the decode bar, and rows that receive nothing stay untouched."""
    fmt, D, I, nr, S, act, a, b, nulls, bad = case
    say("combine", case)
    rng = np.random.default_rng(D * 5 + I + 3)
    c = random_case(rng, fmt, D, I, nr, S, act, a, b, nulls, bad)
    exp = oracle_out(orc, c, act, a, b)
    got_a = run_dev(hip, c, act, a, b)
    assert hip.set_option("combine_ordered", 1)
    try:
        got_o = run_dev(hip, c, act, a, b)
    finally:
        hip.set_option("combine_ordered", 0)
    for got in (got_a, got_o):
        assert npref.rel_err(got, exp) < TOL_F32
    touched = set(int(r) for r in c.rows if 0 <= r < c.S)
    for t in range(c.out.shape[0]):
        if t not in touched:
            assert np.array_equal(got_a[t], c.out[t])
    # the host-pointer drop-in always combines in the reference's order: two calls give
    # bit-identical results, equal to the ordered device call's
    h1, h2 = c.out.copy(), c.out.copy()
    hip.moe_block(*c.args(h1), act, a, b)
    hip.moe_block(*c.args(h2), act, a, b)
    assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))
    assert np.array_equal(h1.view(np.uint32), got_o.view(np.uint32))
