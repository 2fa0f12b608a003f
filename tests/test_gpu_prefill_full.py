"""Prefill configurations at their full sizes (c4: T=2048, Zipf(1.1) routing, 16,384 rows,
the heaviest expert ~1,750 rows; c3: T=512, 4,096 rows) through the default path, checked
against the oracle (cpu_moe_block, src/gpu/metal_ops.cpp:278-342) on a deterministic
sample of rows.

Rows of a moe_block call are independent, so the call is run twice on the GPU:
  * with the real combine (rows = tokens, rw = top-k weights, out [T, D]);
  * with an identity combine (row j -> out row j, weight 1), same segments, so out row j
    is expert(j)'s output y_j for xg row j: the grouped GEMM's row classes and blocks are
    exactly those of the real call.
Sampled rows of y are compared with oracle calls of nb = 1 on those rows only: rows
across every 128-row block of the heaviest expert, rows of a mid-size expert, and one
row each of the smallest experts.  The bar is per row (max|y - ref| / max|ref| of that
row) as well as global.  The real call's out is then checked on every token that the
sampled experts' rows reach: the combine applied on the host to the GPU's y rows in the
reference's order (product, then sum) must give the GPU's out bit for bit.
"""
import sys

import numpy as np
import pytest
import torch

import npref

pytestmark = pytest.mark.gpu

TOL_ROW = 1e-2     # bf16 activations in the grouped GEMM (north-star bar for bf16 outputs)
N_SAMPLE = 32


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def sample_rows(nr, xoff, rng):
    """(expert index, rows of that expert) triples: the heaviest expert across all its
    128-row blocks, a mid-size expert, one expert of each size range that a row class of
    its own serves (33-64, 65-128, 129-256 and more rows), and the tail (one row of each of
    the smallest)."""
    order = np.argsort(-nr, kind="stable")
    heavy = int(order[0])
    n_h = int(nr[heavy])
    picks = {heavy: sorted(set(np.linspace(0, n_h - 1, N_SAMPLE).round().astype(int).tolist()
                               + [min(n_h - 1, 128 * b + 127) for b in range((n_h + 127) // 128)]))}
    mid = int(order[len(order) // 8])
    n_m = int(nr[mid])
    picks[mid] = sorted(rng.choice(n_m, size=min(N_SAMPLE, n_m), replace=False).tolist())
    for lo, hi in ((33, 64), (65, 128), (129, 256), (257, 1 << 30)):
        for e in order:
            e = int(e)
            if lo <= int(nr[e]) <= hi and e not in picks:
                n_e = int(nr[e])
                # its first and last rows, and rows between
                picks[e] = sorted(set([0, n_e - 1] + rng.choice(
                    n_e, size=min(N_SAMPLE // 2, n_e), replace=False).tolist()))
                break
    for e in order[::-1][:N_SAMPLE]:
        e = int(e)
        if e not in picks:
            picks[e] = [int(rng.integers(0, int(nr[e])))]
    return picks


@pytest.mark.parametrize("name,T", [("c4", 2048), ("c3", 512)])
def test_prefill_full_size(hip, orc, name, T):
    from mvllm_hip import synth
    say("prefill full size", name, T)
    w = synth.make_workload(name, T=T, with_experts=False)
    D, I, fmt = w.D, w.I, w.fmt
    R = int(w.nr.sum())
    geom = hip.expert_geom(fmt, D, I)
    pool, stride = synth.device_pool(torch, fmt, D, I, w.nb, 4321 + T, geom)
    off = geom[1]
    base = pool.data_ptr()
    order = (0, 2, 4, 1, 3, 5)
    ptrs = [[base + i * stride + int(off[o]) for i in range(w.nb)] for o in order]
    say("  experts", w.nb, "rows", R, "largest", int(w.nr.max()), "median",
        int(np.median(w.nr)))
    if name == "c4":
        assert int(w.nr.max()) > 14 * 128 - 128  # the heavy expert spans 14 row blocks
    xg = torch.from_numpy(w.xg).cuda()
    # identity combine: out row j = y_j
    y = torch.zeros((R, D), dtype=torch.float32, device="cuda")
    hip.moe_block_dev(w.nb, D, I, fmt, *ptrs, xg, w.xoff, w.nr, np.arange(R, dtype=np.int32),
                      np.ones(R, np.float32), y, R, w.act, w.a, w.b)
    # the real call
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    hip.moe_block_dev(w.nb, D, I, fmt, *ptrs, xg, w.xoff, w.nr, w.rows, w.rw, out, T, w.act,
                      w.a, w.b)
    torch.cuda.synchronize()
    rng = np.random.default_rng(11)
    picks = sample_rows(w.nr, w.xoff, rng)
    worst, errs, n_rows = 0.0, [], 0
    ys = {}
    for e, rs in picks.items():
        j = int(w.xoff[e]) + np.asarray(rs, np.int64)
        gp, up, dp, gs, us, ds = synth.blob_pieces(pool[e].cpu().numpy(), fmt, D, I, off)
        exp = np.zeros((len(rs), D), np.float32)
        assert orc.moe_block(1, D, I, fmt, [gp], [up], [dp], [gs], [us], [ds], w.xg[j],
                             np.zeros(1, np.int32), np.array([len(rs)], np.int32),
                             np.arange(len(rs), dtype=np.int32), np.ones(len(rs), np.float32),
                             exp, len(rs), w.act, w.a, w.b) == 1
        got = y[torch.from_numpy(j).cuda()].cpu().numpy()
        for r in range(len(rs)):
            err = npref.rel_err(got[r], exp[r])
            errs.append(err)
            worst = max(worst, err)
            ys[int(j[r])] = got[r]
        n_rows += len(rs)
        if len(rs) > 1:
            say(f"  expert {e}: {int(w.nr[e])} rows, {len(rs)} sampled, worst row "
                f"{max(errs[-len(rs):]):.2e}")
    say(f"  {n_rows} rows of {len(picks)} experts: worst per-row rel err {worst:.2e}, "
        f"median {np.median(errs):.2e}")
    assert worst < TOL_ROW
    # the real call's combine, on tokens whose every row was sampled... every token has 8
    # rows, so instead: all tokens reached by the sampled rows, with the GPU's own y rows
    # (from the identity call) for all their entries, in the reference's order
    yall = y.cpu().numpy()
    outg = out.cpu().numpy()
    toks = sorted(set(int(w.rows[j]) for j in ys))[:64]
    by_tok = {t: [] for t in toks}
    for j in range(R):  # compact rows in expert order
        t = int(w.rows[j])
        if t in by_tok:
            by_tok[t].append(j)
    for t in toks:
        acc = np.zeros(D, np.float32)
        for j in by_tok[t]:
            acc = (acc + (np.float32(w.rw[j]) * yall[j]).astype(np.float32)).astype(np.float32)
        assert np.array_equal(acc.view(np.uint32), outg[t].view(np.uint32)), t
    say(f"  combine bit-exact on {len(toks)} tokens")


def test_prefill_full_size_fp4act(hip, orc):
    """c4 at its full size with native MXFP4 activations (option fp4act): experts of more
    than 32 rows through the scaled-FP4 kernel in 256-row blocks, each remainder in the
    smallest of the 64-, 128- and 256-row classes that holds it; the 16/32-row classes
    through the bf16 GEMM on exact bf16 copies of the quantized activations.  Sampled rows
    (as above, an expert of each class among them) against the composed oracle
    (fp4_activation_qdq on x and H around the f32 moe_block maths, nb = 1 on those rows),
    with the native-FP4 bar per row (each row's error over its own largest |ref|) and
    over all rows: products are exact, so only the summation order differs, except where
    it moves an h value across an e2m1 rounding boundary (rare; one code step of one h
    element)."""
    from mvllm_hip import synth
    name, T = "c4", 2048
    say("prefill full size fp4act", name, T)
    w = synth.make_workload(name, T=T, with_experts=False)
    D, I, fmt = w.D, w.I, w.fmt
    R = int(w.nr.sum())
    geom = hip.expert_geom(fmt, D, I)
    pool, stride = synth.device_pool(torch, fmt, D, I, w.nb, 4321 + T, geom)
    off = geom[1]
    base = pool.data_ptr()
    order = (0, 2, 4, 1, 3, 5)
    ptrs = [[base + i * stride + int(off[o]) for i in range(w.nb)] for o in order]
    xg = torch.from_numpy(w.xg).cuda()
    y = torch.zeros((R, D), dtype=torch.float32, device="cuda")
    assert hip.set_option("fp4act", 1)
    try:
        hip.moe_block_dev(w.nb, D, I, fmt, *ptrs, xg, w.xoff, w.nr,
                          np.arange(R, dtype=np.int32), np.ones(R, np.float32), y, R, w.act,
                          w.a, w.b)
        torch.cuda.synchronize()
    finally:
        hip.set_option("fp4act", 0)
    rng = np.random.default_rng(12)
    picks = sample_rows(w.nr, w.xoff, rng)
    gots, exps = [], []
    for e, rs in picks.items():
        j = int(w.xoff[e]) + np.asarray(rs, np.int64)
        gp, up, dp, gs, us, ds = synth.blob_pieces(pool[e].cpu().numpy(), fmt, D, I, off)
        exp = np.zeros((len(rs), D), np.float32)
        assert orc.moe_block_fp4act(1, D, I, fmt, [gp], [up], [dp], [gs], [us], [ds], w.xg[j],
                                    np.zeros(1, np.int32), np.array([len(rs)], np.int32),
                                    np.arange(len(rs), dtype=np.int32),
                                    np.ones(len(rs), np.float32), exp, len(rs), w.act, w.a,
                                    w.b) == 1
        gots.append(y[torch.from_numpy(j).cuda()].cpu().numpy())
        exps.append(exp)
    got, exp = np.concatenate(gots), np.concatenate(exps)
    den = np.max(np.abs(exp))
    dev_ = np.abs(got.astype(np.float64) - exp) / den
    # per row: over the row's own largest |ref| (floored at 1e-3 of the global one, for a
    # row whose reference is all but zero)
    den_r = np.maximum(np.max(np.abs(exp), axis=1, keepdims=True), 1e-3 * den)
    row_err = np.max(np.abs(got.astype(np.float64) - exp) / den_r, axis=1)
    say(f"  {got.shape[0]} rows of {len(picks)} experts: rel_err max {float(dev_.max()):.2e}, "
        f"p99 {float(np.quantile(dev_, 0.99)):.2e}, worst row {float(row_err.max()):.2e}")
    assert float(row_err.max()) < TOL_ROW
    assert float(dev_.max()) < 1e-2
    assert float(np.quantile(dev_, 0.99)) < 1e-5
