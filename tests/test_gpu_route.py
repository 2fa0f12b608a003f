"""GPU parity of the device routing (mvllm_hip_moe_topk_dev, mvllm_hip_moe_segments_dev)
against the oracle's moe_topk / moe_segments (which the oracle tests pin to the
reference's known answers and to the reference build).  Bar: bit-exact ids, offsets,
counts and f32 weights."""
import ctypes
import zlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_topk(hip, choice, mix, k):
    T, E = choice.shape
    idx = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
    wt = torch.zeros((T, k), dtype=torch.float32, device="cuda")
    hip.moe_topk_dev(dev(choice), None if mix is None else dev(mix), T, E, k, idx, wt)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), wt.cpu().numpy()


def check_topk(orc, choice, mix, k, gi, gw):
    for t in range(choice.shape[0]):
        kk, ei, ew = orc.moe_topk(choice[t], k, None if mix is None else mix[t])
        assert kk == k
        assert np.array_equal(gi[t], ei), (t, gi[t], ei)
        assert np.array_equal(gw[t].view(np.uint32), ew.view(np.uint32)), (t, gw[t], ew)


def topk_case(name):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    if name == "c4":        # K3 routing shape, scores with many exact ties
        T, E, k = 64, 384, 8
        choice = (np.round(rng.standard_normal((T, E)) * 4) / 4).astype(np.float32)
        mix = rng.standard_normal((T, E)).astype(np.float32)  # negatives clip to 0
    elif name == "c1":      # OLMoE shape, weights from the scores themselves
        T, E, k = 33, 64, 8
        choice = rng.standard_normal((T, E)).astype(np.float32)
        choice[3] = -np.abs(choice[3])  # all picks negative: uniform 1/k
        mix = None
    elif name == "k_eq_n":
        T, E, k = 5, 7, 7
        choice = rng.integers(-2, 3, size=(T, E)).astype(np.float32)
        mix = np.abs(rng.standard_normal((T, E))).astype(np.float32)
    elif name == "max":     # 4096 experts, k = 64
        T, E, k = 17, 4096, 64
        choice = rng.standard_normal((T, E)).astype(np.float32)
        choice[:, ::97] = 1.5  # ties across the lanes' strided subsets
        mix = rng.uniform(0, 1, (T, E)).astype(np.float32)
    elif name == "k1":
        T, E, k = 9, 100, 1
        choice = rng.standard_normal((T, E)).astype(np.float32)
        mix = rng.standard_normal((T, E)).astype(np.float32)
    else:                   # signed zeros and infinities
        T, E, k = 4, 70, 6
        choice = np.zeros((T, E), np.float32)
        choice[0, 5] = -0.0
        choice[0, 2] = np.inf
        choice[1, :] = -np.inf
        choice[1, 69] = -1.0
        choice[2, 10:20] = -0.0
        choice[3, 60] = np.inf
        choice[3, 61] = np.inf
        mix = None
    return choice, mix, k


@pytest.mark.parametrize("name", ["c4", "c1", "k_eq_n", "max", "k1", "zeros_inf"])
def test_topk_bit_exact(hip, orc, name):
    choice, mix, k = topk_case(name)
    say("topk", name, choice.shape, k)
    gi, gw = gpu_topk(hip, choice, mix, k)
    check_topk(orc, choice, mix, k, gi, gw)


def gpu_segments(hip, idx, wt, n_exp, cap_experts, cap_rows):
    T, topk = idx.shape
    work = torch.zeros(2 * n_exp + 1, dtype=torch.int32, device="cuda")
    eids = torch.full((cap_experts,), -7, dtype=torch.int32, device="cuda")
    xoff = torch.full((cap_experts,), -7, dtype=torch.int32, device="cuda")
    nr = torch.full((cap_experts,), -7, dtype=torch.int32, device="cuda")
    rows = torch.full((cap_rows,), -7, dtype=torch.int32, device="cuda")
    rw = torch.zeros(cap_rows, dtype=torch.float32, device="cuda")
    counts = torch.full((2,), -9, dtype=torch.int32, device="cuda")
    hip.moe_segments_dev(dev(idx), dev(wt), T, topk, n_exp, work, eids, xoff, nr, rows, rw,
                         counts)
    torch.cuda.synchronize()
    c = counts.cpu().numpy()
    nb, n = int(c[0]), int(c[1])
    if nb < 0:
        return nb, n, None
    return nb, n, (eids.cpu().numpy()[:nb], xoff.cpu().numpy()[:nb], nr.cpu().numpy()[:nb],
                   rows.cpu().numpy()[:n], rw.cpu().numpy()[:n])


def check_segments(orc, idx, wt, got, cap_experts):
    T, topk = idx.shape
    nb, n, arrs = got
    enb, eeids, exoff, enr, erows, erw = orc.moe_segments(idx, wt, T, topk, cap_experts)
    assert nb == enb and n == len(erows)
    g_eids, g_xoff, g_nr, g_rows, g_rw = arrs
    assert np.array_equal(g_eids, eeids)
    assert np.array_equal(g_xoff, exoff)
    assert np.array_equal(g_nr, enr)
    assert np.array_equal(g_rows, erows)
    assert np.array_equal(g_rw.view(np.uint32), erw.view(np.uint32))


def test_route_then_segments(hip, orc):
    """The batched-call arguments of a K3-shaped layer, all on the device."""
    rng = np.random.default_rng(11)
    T, E, k = 512, 384, 8
    choice = rng.standard_normal((T, E)).astype(np.float32)
    choice += np.log(1 + np.arange(E, dtype=np.float32))[::-1] * 0.5  # skewed popularity
    mix = (1 / (1 + np.exp(-choice))).astype(np.float32)
    gi, gw = gpu_topk(hip, choice, mix, k)
    check_topk(orc, choice, mix, k, gi, gw)
    got = gpu_segments(hip, gi, gw, E, E, T * k)
    say("route: nb", got[0], "rows", got[1])
    check_segments(orc, gi, gw, got, E)


@pytest.mark.parametrize("T,topk,E", [(50, 6, 20), (1, 8, 64), (700, 3, 1500)])
def test_segments_arbitrary_ids(hip, orc, T, topk, E):
    """ids with -1 entries, an expert twice in one token, zero and cancelling weights."""
    rng = np.random.default_rng(T * 7 + E)
    idx = rng.integers(-1, E, size=(T, topk)).astype(np.int32)
    wt = rng.standard_normal((T, topk)).astype(np.float32)
    wt[rng.random((T, topk)) < 0.15] = 0.0
    if topk >= 2:
        idx[::5, 1] = idx[::5, 0]          # duplicate pick: weights add in slot order
        wt[::10, 1] = -wt[::10, 0]         # ... and sometimes cancel to 0 (row dropped)
    got = gpu_segments(hip, idx, wt, E, E, T * topk)
    say("segments", T, topk, E, "nb", got[0], "rows", got[1])
    check_segments(orc, idx, wt, got, E)


def test_segments_caps_and_bad_ids(hip, orc):
    rng = np.random.default_rng(5)
    T, topk, E = 200, 4, 40
    idx = rng.integers(0, E, size=(T, topk)).astype(np.int32)
    wt = rng.uniform(0.1, 1.0, size=(T, topk)).astype(np.float32)
    # union truncated to the 10 smallest ids, as the host union does
    got = gpu_segments(hip, idx, wt, E, 10, T * topk)
    check_segments(orc, idx, wt, got, 10)
    # rows one short: -1, like the host function
    full = gpu_segments(hip, idx, wt, E, E, T * topk)
    short = gpu_segments(hip, idx, wt, E, E, full[1] - 1)
    assert short[0] == -1 and short[1] == -1
    # the host function with the same short capacity also returns -1
    cap = full[1] - 1
    bufs = [np.zeros(E, np.int32) for _ in range(3)] + [np.zeros(cap, np.int32),
                                                         np.zeros(cap, np.float32)]
    n = ctypes.c_int(0)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert orc.lib.orc_moe_segments(P(idx), P(wt), T, topk, *[P(b) for b in bufs], E, cap,
                                    ctypes.cast(ctypes.pointer(n), ctypes.c_void_p)) == -1
    # an id outside [0, n_exp): reported, not counted
    bad = idx.copy()
    bad[7, 2] = E
    assert gpu_segments(hip, bad, wt, E, E, T * topk)[0] == -1


@pytest.mark.parametrize("T,E,k", [(16, 64, 8), (1, 384, 8), (512, 384, 8), (2048, 384, 8),
                                   (40, 1024, 64), (30, 2000, 3)])
def test_route_dev(hip, orc, T, E, k):
    """mvllm_hip_moe_route_dev (top-k and segments in one call) against the oracle's
    moe_topk per token and moe_segments of its picks."""
    rng = np.random.default_rng(T * 13 + E + k)
    choice = (np.round(rng.standard_normal((T, E)) * 8) / 8).astype(np.float32)
    mix = rng.standard_normal((T, E)).astype(np.float32) if k != 3 else None
    i32 = dict(dtype=torch.int32, device="cuda")
    idx, wt = torch.full((T, k), -7, **i32), torch.zeros((T, k), dtype=torch.float32, device="cuda")
    work, counts = torch.zeros(2 * E + 1, **i32), torch.full((2,), -9, **i32)
    eids, xoff, nr = (torch.full((E,), -7, **i32) for _ in range(3))
    rows, rw = torch.full((T * k,), -7, **i32), torch.zeros(T * k, dtype=torch.float32, device="cuda")
    hip.moe_route_dev(dev(choice), None if mix is None else dev(mix), T, E, k, idx, wt, work,
                      eids, xoff, nr, rows, rw, counts)
    torch.cuda.synchronize()
    gi, gw = idx.cpu().numpy(), wt.cpu().numpy()
    check_topk(orc, choice, mix, k, gi, gw)
    nb, n = (int(v) for v in counts.cpu().numpy())
    say("route_dev", T, E, k, "nb", nb, "rows", n)
    got = (nb, n, (eids.cpu().numpy()[:nb], xoff.cpu().numpy()[:nb], nr.cpu().numpy()[:nb],
                   rows.cpu().numpy()[:n], rw.cpu().numpy()[:n]))
    check_segments(orc, gi, gw, got, E)



@pytest.mark.parametrize("fmt,D,I,T,E,k", [(4, 512, 256, 16, 64, 8), (7, 1024, 512, 6, 48, 4)])
def test_route_feeds_moe_block(hip, orc, fmt, D, I, T, E, k):
    """One layer batched the way a GPU-resident caller would run it: device routing, its
    segments and the gathered token rows into one mvllm_hip_moe_block_dev call, against
    the oracle's host chain (moe_topk per token, moe_segments, moe_block)."""
    from cases import expert_arrays
    from mvllm_hip import ACT_CLAMP_SWIGLU, ACT_SITU
    rng = np.random.default_rng(D + T * E)
    ex = [expert_arrays(rng, fmt, D, I) for _ in range(E)]
    X = rng.standard_normal((T, D)).astype(np.float32)
    choice = rng.standard_normal((T, E)).astype(np.float32)
    mix = (1 / (1 + np.exp(-choice))).astype(np.float32)
    act, a, b = (ACT_CLAMP_SWIGLU, 7.0, 0.0) if fmt == 4 else (ACT_SITU, 4.0, 25.0)
    # device: route, then one batched call
    i32 = dict(dtype=torch.int32, device="cuda")
    idx, wt = torch.empty((T, k), **i32), torch.empty((T, k), dtype=torch.float32, device="cuda")
    work, counts = torch.zeros(2 * E + 1, **i32), torch.empty(2, **i32)
    eids, xoff, nr = (torch.empty(E, **i32) for _ in range(3))
    rows, rw = torch.empty(T * k, **i32), torch.empty(T * k, dtype=torch.float32, device="cuda")
    hip.moe_route_dev(dev(choice), dev(mix), T, E, k, idx, wt, work, eids, xoff, nr, rows, rw,
                      counts)
    torch.cuda.synchronize()
    nb, n = (int(v) for v in counts.cpu().numpy())
    g_eids, g_xoff, g_nr = (x.cpu().numpy()[:nb] for x in (eids, xoff, nr))
    g_rows, g_rw = rows.cpu().numpy()[:n], rw.cpu().numpy()[:n]
    keep = []

    def L(key):
        out = []
        for e in g_eids:
            t = dev(ex[e][key])
            keep.append(t)
            out.append(t.data_ptr())
        return out
    lists = [L(key) for key in ("gp", "up", "dp", "gs", "us", "ds")]
    xg = dev(X[g_rows])
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    hip.moe_block_dev(nb, D, I, fmt, *lists, xg, g_xoff, g_nr, g_rows, g_rw, out, T, act, a, b)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    # host: the reference chain on the same scores
    hi = np.zeros((T, k), np.int32)
    hw = np.zeros((T, k), np.float32)
    for t in range(T):
        _, hi[t], hw[t] = orc.moe_topk(choice[t], k, mix[t])
    enb, e_eids, e_xoff, e_nr, e_rows, e_rw = orc.moe_segments(hi, hw, T, k, E)
    assert enb == nb and np.array_equal(e_eids, g_eids) and np.array_equal(e_rows, g_rows)
    exp = np.zeros((T, D), np.float32)
    sel = [ex[e] for e in e_eids]
    assert orc.moe_block(enb, D, I, fmt, *[[s[key] for s in sel] for key in
                                           ("gp", "up", "dp", "gs", "us", "ds")],
                         X[e_rows], e_xoff, e_nr, e_rows, e_rw, exp, T, act, a, b) == 1
    import npref
    err = npref.rel_err(got, exp)
    say("route -> moe_block", fmt, "nb", nb, "rows", n, "rel_err", err)
    assert err < 2e-5
