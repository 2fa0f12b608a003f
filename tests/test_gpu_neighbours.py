"""GPU parity of the steps either side of the routed block: fmt 0 (f32) experts on the f32
matrix cores (the shared experts, src/model/kimi_k3.cpp:192-209), the router
(cpu_route, src/gpu/metal_ops.cpp:213-231), dense linears (QuantMat::gemm,
src/quant/weight.cpp:47-64; K3's latent down / up, src/model/kimi_k3.cpp:2003-2006,
2074-2090), RMSNorm (quant::rmsnorm, src/quant/quant.cpp:384-398) and a K3-shaped chain of
them around moe_block, against the CPU oracle (pinned to the reference build by the CPU
suite).

Bars: f32 arithmetic in another summation order, 2e-5 relative (max|y - ref| / max|ref|);
linears on int4 / MXFP4 weights take their input rows as two bf16 terms (2^-17), 1e-4.
Router: the device's dot products and expf may move a score by a few ulp, so picks must
agree wherever the host's k-th and (k+1)-th choices are more than 1e-5 (relative) apart,
and the weights of agreeing tokens within 1e-5.
"""
import sys

import numpy as np
import pytest
import torch

import npref
from cases import expert_arrays, random_case

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_block(hip, c):
    keep = []

    def L(xs):
        if xs is None:
            return None
        out = []
        for x in xs:
            t = None if x is None else dev(x)
            keep.append(t)
            out.append(None if t is None else t.data_ptr())
        return out
    lists = [L(c.g), L(c.u), L(c.d), L(c.gs), L(c.us), L(c.ds)]
    out = dev(c.out)
    hip.moe_block_dev(c.nb, c.D, c.I, c.fmt, *lists, dev(c.xg), c.xoff, c.nr, c.rows, c.rw, out,
                      c.S, c.act, c.a, c.b)
    torch.cuda.synchronize()
    return out.cpu().numpy()


F32_CASES = [
    # D, I, nr, S, act, a, b
    (512, 256, [1, 2, 3], 6, 1, 7.0, 0.0),          # decode rows, ClampSwiGLU
    (7168, 2048, [1], 1, 2, 4.0, 25.0),             # K3 shared expert (SiTU), one token
    (6144, 2048, [3], 3, 1, 7.0, 0.0),              # GLM shared expert shape
    (1024, 512, [40, 5, 70], 80, 0, 0.0, 0.0),      # prefill rows: 16-, 32- and 64-row items
]


@pytest.mark.parametrize("case", F32_CASES)
def test_fmt0_block_on_f32_matrix_cores(hip, orc, case):
    D, I, nr, S, act, a, b = case
    say("fmt0 block", case)
    rng = np.random.default_rng(D + I + len(nr))
    c = random_case(rng, 0, D, I, nr, S, act, a, b)
    hip.stats_reset()
    got = run_block(hip, c)
    st = hip.stats()
    exp = c.out.copy()
    assert orc.moe_block(*c.args(exp), act, a, b) == 1
    err = npref.rel_err(got, exp)
    say("  rel_err", err, "launches", st["launches_gate_up"], st["launches_down"])
    assert err < TOL_F32


@pytest.mark.parametrize("T,D,E,k,rscale,bias", [(1, 7168, 384, 8, 2.5, True),
                                                 (16, 2048, 64, 8, 1.0, False),
                                                 (300, 1024, 256, 8, 1.0, True)])
def test_router_matches_host_router(hip, orc, T, D, E, k, rscale, bias):
    say("router", T, D, E, k)
    rng = np.random.default_rng(T + D + E)
    x = rng.standard_normal((T, D)).astype(np.float32)
    w = (rng.standard_normal((E, D)) * (1.0 / np.sqrt(D))).astype(np.float32)
    bv = (rng.standard_normal(E) * 0.05).astype(np.float32) if bias else None
    f32 = dict(dtype=torch.float32, device="cuda")
    scores, choice = torch.empty((T, E), **f32), torch.empty((T, E), **f32)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    wt = torch.empty((T, k), **f32)
    hip.router_dev(dev(x), dev(w), None if bv is None else dev(bv), T, D, E, k, rscale, scores,
                   choice, idx, wt)
    torch.cuda.synchronize()
    gi, gw = idx.cpu().numpy(), wt.cpu().numpy()
    ei, ew = orc.route(x, w, bv, k, rscale)
    # the host's choices in f64, for the gap between the k-th and (k+1)-th
    s64 = x.astype(np.float64) @ w.astype(np.float64).T
    ch = 1.0 / (1.0 + np.exp(-s64)) + (0.0 if bv is None else bv.astype(np.float64))
    srt = -np.sort(-ch, axis=1)
    gap = (srt[:, k - 1] - srt[:, k]) / np.maximum(np.abs(srt[:, k - 1]), 1e-30)
    clear = gap > 1e-5
    # as sets (two picks a few ulp apart inside the top k may swap places), weights matched
    # by expert id
    go, eo = np.argsort(gi, axis=1, kind="stable"), np.argsort(ei, axis=1, kind="stable")
    gi_s, ei_s = np.take_along_axis(gi, go, 1), np.take_along_axis(ei, eo, 1)
    gw_s, ew_s = np.take_along_axis(gw, go, 1), np.take_along_axis(ew, eo, 1)
    agree = np.all(gi_s == ei_s, axis=1)
    in_order = np.all(gi == ei, axis=1)
    say(f"  tokens {T}: clear {int(clear.sum())}, picks agree {int(agree.sum())}, same order "
        f"{int(in_order.sum())}")
    assert np.all(agree[clear])
    assert np.max(np.abs(gw_s[agree] - ew_s[agree]) /
                  np.maximum(np.abs(ew_s[agree]), 1e-30)) < 1e-5


@pytest.mark.parametrize("fmt,O,K,n", [(0, 2048, 7168, 1), (0, 7168, 2048, 5), (0, 64, 48, 3),
                                       (4, 2048, 6144, 1), (4, 512, 1024, 40),
                                       (7, 7168, 2048, 3), (7, 256, 512, 70),
                                       (8, 2048, 7168, 1), (8, 7168, 2048, 4),
                                       (8, 7168, 7168, 1), (8, 96, 48, 37)])
def test_linear(hip, orc, fmt, O, K, n):
    """fmt 8 (QuantMat's int8 rows, MVLLM_DENSE_BITS=8) at K3's latent shapes, with codes
    and scales from the reference's quantizer rule (row amax / 127, clamp +-127) and an
    all-zero row (scale 0)."""
    say("linear", fmt, O, K, n)
    rng = np.random.default_rng(O + K + n + fmt)
    x = rng.standard_normal((n, K)).astype(np.float32)
    if fmt == 0:
        w = (rng.standard_normal((O, K)) * 0.05).astype(np.float32)
        sc = None
    elif fmt == 8:
        wf = (rng.standard_normal((O, K)) * 0.05).astype(np.float32)
        wf[1] = 0.0
        amax = np.abs(wf).max(axis=1)
        sc = (amax / np.float32(127.0)).astype(np.float32)
        inv = np.where(sc > 0, np.float32(1.0) / np.where(sc > 0, sc, 1), 0).astype(np.float32)
        w = np.clip(np.round(wf * inv[:, None]), -127, 127).astype(np.int8)
    else:
        e = expert_arrays(rng, fmt, K, O)   # gate: [O, K] codes and scales
        w, sc = e["gp"], e["gs"]
    y = torch.zeros((n, O), dtype=torch.float32, device="cuda")
    hip.linear_dev(fmt, dev(w), None if sc is None else dev(sc), O, K, dev(x), n, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    exp = orc.matmul(fmt, x, w, sc)
    err = npref.rel_err(got, exp)
    say("  rel_err", err)
    assert err < (TOL_F32 if fmt in (0, 8) else 1e-4)


def test_linear_refuses_odd_shapes(hip):
    """Shapes and formats the kernels do not take return 0 (the host runs them), with a
    message."""
    buf = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    assert hip.lib().mvllm_hip_linear_dev(8, buf.data_ptr(), buf.data_ptr(), 100, 256,
                                          buf.data_ptr(), 1, buf.data_ptr(), None) == 0
    assert hip.lib().mvllm_hip_linear_dev(8, buf.data_ptr(), None, 256, 256,
                                          buf.data_ptr(), 1, buf.data_ptr(), None) == 0
    assert hip.lib().mvllm_hip_linear_dev(5, buf.data_ptr(), buf.data_ptr(), 256, 256,
                                          buf.data_ptr(), 1, buf.data_ptr(), None) == 0
    assert hip.lib().mvllm_hip_linear_dev(4, buf.data_ptr(), buf.data_ptr(), 100, 256,
                                          buf.data_ptr(), 1, buf.data_ptr(), None) == 0
    assert b"linear_dev" in hip.lib().mvllm_hip_last_error()


@pytest.mark.parametrize("rows,n,with_w", [(1, 7168, True), (9, 2048, True), (4, 333, False)])
def test_rmsnorm(hip, orc, rows, n, with_w):
    say("rmsnorm", rows, n)
    rng = np.random.default_rng(rows + n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32) if with_w else None
    y = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    hip.rmsnorm_dev(dev(x), None if w is None else dev(w), y, rows, n, 1e-6)
    torch.cuda.synchronize()
    err = npref.rel_err(y.cpu().numpy(), orc.rmsnorm(x, w, 1e-6))
    say("  rel_err", err)
    assert err < 2e-6


def test_k3_latent_chain(hip, orc):
    """K3's routed MoE around the block (src/model/kimi_k3.cpp:1973-2090) on the device:
    router on x -> top-k -> segments; z = lat_down(x) (int4); the batched block on z rows
    (MXFP4 experts, SiTU); acc -> rmsnorm(lat_n) -> lat_up (f32) -> uph.  The oracle runs
    the same chain from the device's routing (routing parity is the test above)."""
    say("k3 chain")
    rng = np.random.default_rng(2090)
    T, H, L, I, E, k = 12, 1024, 512, 256, 32, 4
    x = rng.standard_normal((T, H)).astype(np.float32)
    w_r = (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float32)
    dn = expert_arrays(rng, 4, H, L)                      # lat_down: [L, H] int4-g64
    w_up = (rng.standard_normal((H, L)) * 0.05).astype(np.float32)   # lat_up: f32 [H, L]
    lat_n = rng.uniform(0.5, 1.5, L).astype(np.float32)
    experts = [expert_arrays(rng, 7, L, I) for _ in range(E)]
    f32 = dict(dtype=torch.float32, device="cuda")
    i32 = dict(dtype=torch.int32, device="cuda")
    # router -> segments
    scores, choice = torch.empty((T, E), **f32), torch.empty((T, E), **f32)
    idx, wt = torch.empty((T, k), **i32), torch.empty((T, k), **f32)
    hip.router_dev(dev(x), dev(w_r), None, T, H, E, k, 1.0, scores, choice, idx, wt)
    work, counts = torch.empty(2 * E + 1, **i32), torch.empty(2, **i32)
    eids, xoff, nr = (torch.empty(E, **i32) for _ in range(3))
    rows, rw = torch.empty(T * k, **i32), torch.empty(T * k, **f32)
    hip.moe_segments_dev(idx, wt, T, k, E, work, eids, xoff, nr, rows, rw, counts)
    # z = lat_down(x)
    z = torch.empty((T, L), **f32)
    hip.linear_dev(4, dev(dn["gp"]), dev(dn["gs"]), L, H, dev(x), T, z)
    torch.cuda.synchronize()
    nb, n_rows = (int(v) for v in counts.cpu())
    e_ids = eids.cpu().numpy()[:nb]
    xo, n_r = xoff.cpu().numpy()[:nb], nr.cpu().numpy()[:nb]
    rws, rwv = rows.cpu().numpy()[:n_rows], rw.cpu().numpy()[:n_rows]
    zg = z[torch.from_numpy(rws.astype(np.int64)).cuda()].contiguous()
    keep = []

    def L_(key):
        out = []
        for e in e_ids:
            t = dev(experts[int(e)][key])
            keep.append(t)
            out.append(t.data_ptr())
        return out
    acc = torch.zeros((T, L), **f32)
    hip.moe_block_dev(nb, L, I, 7, L_("gp"), L_("up"), L_("dp"), L_("gs"), L_("us"), L_("ds"),
                      zg, xo, n_r, rws, rwv, acc, T, 2, 4.0, 25.0)
    accn = torch.empty((T, L), **f32)
    hip.rmsnorm_dev(acc, dev(lat_n), accn, T, L, 1e-6)
    uph = torch.empty((T, H), **f32)
    hip.linear_dev(0, dev(w_up), None, H, L, accn, T, uph)
    torch.cuda.synchronize()
    got = uph.cpu().numpy()
    # the oracle chain, from the device's routing
    z_o = orc.matmul(4, x, dn["gp"], dn["gs"])
    ex = [experts[int(e)] for e in e_ids]
    acc_o = np.zeros((T, L), np.float32)
    assert orc.moe_block(nb, L, I, 7, [e["gp"] for e in ex], [e["up"] for e in ex],
                         [e["dp"] for e in ex], [e["gs"] for e in ex], [e["us"] for e in ex],
                         [e["ds"] for e in ex], np.ascontiguousarray(z_o[rws]), xo, n_r, rws,
                         rwv, acc_o, T, 2, 4.0, 25.0) == 1
    uph_o = orc.matmul(0, orc.rmsnorm(acc_o, lat_n, 1e-6), w_up)
    err = npref.rel_err(got, uph_o)
    say("  rel_err", err)
    assert err < 1e-4
