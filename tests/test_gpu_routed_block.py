"""The device-resident layer (mvllm_hip_moe_block_routed_dev): routing on the device, then
the block on the segments where the routing left them, experts resolved through a device
blob table; no host round trip (src/model/glm53.cpp:1938-1992 with the device route).

Two paths: calls of at most 16 out rows run the decode kernels on descriptors the device
planner writes, others the grouped GEMM.  Checked against
  * the host-planned call on the same segments (read back) with the same arithmetic
    (grouped GEMM and same bf16 terms; or the decode kernels with the same K split, the
    same packed or unpacked form and the ordered combine on both sides): bit for bit,
    since items compute rows independently and both combines sum in the reference's
    expert order (decode calls of 9-16 out rows, packed on one side only: within 2e-6);
  * the oracle's host chain (moe_topk per token, moe_segments, moe_block) within the
    arithmetic's bar: 2e-5 for two bf16 terms per activation, 1e-2 (the north-star bar for
    bf16 outputs) for one;
  * the oracle's moe_block on hand-made segments the decode path must split (more rows
    than out rows) and rows whose out row is out of range (skipped), with the combine
    folded into the down kernel (float atomics) and ordered.
Also: null and out-of-table experts consume their rows without writing, and calls whose
caps exceed the routed sizes (surplus workgroups exit) give the same bits.
"""
import sys

import numpy as np
import pytest
import torch

import npref

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def layer(hip, fmt, D, I, T, E, k, seed, null_ids=(), routing="uniform"):
    from mvllm_hip import synth
    rng = np.random.default_rng(seed)
    geom = hip.expert_geom(fmt, D, I)
    pool, stride = synth.device_pool(torch, fmt, D, I, E, seed, geom)
    X = rng.standard_normal((T, D)).astype(np.float32)
    if routing == "skewed":  # a few hot experts: segments of many rows
        bias = np.zeros(E, np.float32)
        bias[:3] = 4.0
        choice = (rng.standard_normal((T, E)) + bias).astype(np.float32)
    else:
        choice = rng.standard_normal((T, E)).astype(np.float32)
    mix = (1 / (1 + np.exp(-choice))).astype(np.float32)
    table = np.array([pool.data_ptr() + e * stride for e in range(E)], np.uint64)
    for e in null_ids:
        table[e] = 0
    return rng, pool, stride, geom, X, choice, mix, table


def route(hip, choice, mix, k, cap_rows=None, cap_e=None):
    T, E = choice.shape
    i32 = dict(dtype=torch.int32, device="cuda")
    idx, wt = torch.empty((T, k), **i32), torch.empty((T, k), dtype=torch.float32, device="cuda")
    work, counts = torch.zeros(2 * E + 1, **i32), torch.empty(2, **i32)
    ce, cr = cap_e or E, cap_rows or T * k
    eids, xoff, nr = (torch.zeros(ce, **i32) for _ in range(3))
    rows, rw = torch.zeros(cr, **i32), torch.zeros(cr, dtype=torch.float32, device="cuda")
    hip.moe_route_dev(dev(choice), dev(mix), T, E, k, idx, wt, work, eids, xoff, nr, rows, rw,
                      counts)
    return counts, eids, xoff, nr, rows, rw


def run_routed(hip, fmt, D, I, table, seg, X, T, act, a, b):
    counts, eids, xoff, nr, rows, rw = seg
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    hip.moe_block_routed_dev(D, I, fmt, dev(table.view(np.int64)), len(table), counts, eids,
                             xoff, nr, rows, rw, dev(X), out, T, act, a, b, status=status)
    torch.cuda.synchronize()
    return out.cpu().numpy(), int(status.cpu()[0])


def host_planned(hip, fmt, D, I, pool, stride, geom, seg, X, T, act, a, b, table):
    counts, eids, xoff, nr, rows, rw = seg
    nb, n = (int(v) for v in counts.cpu().numpy())
    g_eids, g_xoff, g_nr = (t.cpu().numpy()[:nb] for t in (eids, xoff, nr))
    g_rows, g_rw = rows.cpu().numpy()[:n], rw.cpu().numpy()[:n]
    off = geom[1]
    order = (0, 2, 4, 1, 3, 5)
    ptrs = [[(int(table[e]) + int(off[o])) if table[e] else None for e in g_eids]
            for o in order]
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    hip.moe_block_dev(nb, D, I, fmt, *ptrs, dev(X[g_rows]), g_xoff, g_nr, g_rows, g_rw, out, T,
                      act, a, b)
    torch.cuda.synchronize()
    return out.cpu().numpy(), (nb, g_eids, g_xoff, g_nr, g_rows, g_rw)


def oracle_chain(orc, fmt, D, I, pool, stride, geom, choice, mix, k, X, T, act, a, b,
                 null_ids=()):
    from mvllm_hip import synth
    E = choice.shape[1]
    hi = np.zeros((T, k), np.int32)
    hw = np.zeros((T, k), np.float32)
    for t in range(T):
        _, hi[t], hw[t] = orc.moe_topk(choice[t], k, mix[t])
    enb, e_eids, e_xoff, e_nr, e_rows, e_rw = orc.moe_segments(hi, hw, T, k, E)
    blobs = {int(e): pool[int(e)].cpu().numpy() for e in e_eids}
    lists = [[], [], [], [], [], []]
    for e in e_eids:
        pieces = synth.blob_pieces(blobs[int(e)], fmt, D, I, geom[1])
        for j in range(6):
            lists[j].append(None if int(e) in null_ids else pieces[j])
    exp = np.zeros((T, D), np.float32)
    assert orc.moe_block(enb, D, I, fmt, *lists, X[e_rows], e_xoff, e_nr, e_rows, e_rw, exp, T,
                         act, a, b) == 1
    return exp


CASES = [
    # fmt, D, I, T, E, k, routing, path
    (7, 1024, 512, 6, 48, 4, "uniform", "decode"),   # <= 16 out rows: the decode kernels
    (4, 1024, 512, 16, 64, 8, "uniform", "decode"),
    (7, 4096, 512, 8, 64, 8, "uniform", "decode"),    # items of 4 rows: 8 rows do not fit
    (4, 512, 256, 16, 64, 8, "uniform", "gemm"),     # down K = 256: no decode kernel fits
    (7, 512, 256, 300, 64, 8, "skewed", "gemm"),     # > 256 rows: one term; hot experts
]


def set_options(hip, **kv):
    for key, v in kv.items():
        hip.set_option(key, v)


@pytest.mark.parametrize("case", CASES)
def test_routed_block(hip, orc, case):
    fmt, D, I, T, E, k, routing, path = case
    say("routed block", case)
    from mvllm_hip import ACT_CLAMP_SWIGLU, ACT_SITU
    act, a, b = (ACT_CLAMP_SWIGLU, 7.0, 0.0) if fmt == 4 else (ACT_SITU, 4.0, 25.0)
    rng, pool, stride, geom, X, choice, mix, table = layer(hip, fmt, D, I, T, E, k, 17 + T,
                                                          routing=routing)
    seg = route(hip, choice, mix, k)
    got, status = run_routed(hip, fmt, D, I, table, seg, X, T, act, a, b)  # default options
    assert status == 0
    two_terms = T * k <= 256
    if path == "decode":
        # both sides: the decode kernels with one K split, the ordered combine
        set_options(hip, dec_ks=2, combine_ordered=1)
        try:
            got_o, status = run_routed(hip, fmt, D, I, table, seg, X, T, act, a, b)
            ref, info = host_planned(hip, fmt, D, I, pool, stride, geom, seg, X, T, act, a, b,
                                     table)
        finally:
            set_options(hip, dec_ks=0, combine_ordered=0)
        assert status == 0
        if T <= 8:  # both sides run the packed kernels (items of <= 8 rows)
            assert np.array_equal(got_o.view(np.uint32), ref.view(np.uint32))
        else:  # the routed side's items hold up to T rows: the unpacked kernels
            say("  vs host-planned decode: rel", npref.rel_err(got_o, ref))
            assert npref.rel_err(got_o, ref) < 2e-6
        # the default call: its own K split and the folded combine (float atomics, any
        # expert order): the same arithmetic up to summation order
        say("  default vs ordered, split 2: rel", npref.rel_err(got, got_o))
        assert npref.rel_err(got, got_o) < 1e-5
    else:
        # the host-planned call with the same arithmetic: grouped GEMM, same terms
        set_options(hip, gemm=1, mode=1 if two_terms else 0)
        try:
            ref, info = host_planned(hip, fmt, D, I, pool, stride, geom, seg, X, T, act, a, b,
                                     table)
        finally:
            set_options(hip, gemm=0, mode=0)
    nb, _, _, g_nr, _, _ = info
    say(f"  segments {nb}, rows {int(g_nr.sum())}, largest {int(g_nr.max())}")
    if routing == "skewed":
        assert int(g_nr.max()) > 64  # the top row class runs
    if path == "gemm":
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    exp = oracle_chain(orc, fmt, D, I, pool, stride, geom, choice, mix, k, X, T, act, a, b)
    err = npref.rel_err(got, exp)
    say("  rel_err vs oracle chain", err)
    assert err < (2e-5 if two_terms else 1e-2)


def test_routed_block_null_and_missing_experts(hip, orc):
    fmt, D, I, T, E, k = 7, 512, 256, 12, 32, 4
    from mvllm_hip import ACT_SITU
    null_ids = (0, 5, 9)
    rng, pool, stride, geom, X, choice, mix, table = layer(hip, fmt, D, I, T, E, k, 99,
                                                          null_ids=null_ids)
    seg = route(hip, choice, mix, k)
    # the table covers only experts [0, E - 4): the last four are outside it
    short = table[:E - 4]
    got, status = run_routed(hip, fmt, D, I, short, seg, X, T, ACT_SITU, 4.0, 25.0)
    assert status == 0
    gone = set(null_ids) | set(range(E - 4, E))
    exp = oracle_chain(orc, fmt, D, I, pool, stride, geom, choice, mix, k, X, T, ACT_SITU, 4.0,
                       25.0, null_ids=gone)
    err = npref.rel_err(got, exp)
    say("null / missing experts: rel_err", err)
    assert err < 2e-5
    # a misaligned blob address is skipped and reported
    bad = table.copy()
    bad[1] += 16
    got2, status2 = run_routed(hip, fmt, D, I, bad, seg, X, T, ACT_SITU, 4.0, 25.0)
    assert status2 == 2


def test_routed_block_surplus_caps(hip):
    """Caps above the routed sizes (the grid sized for them, surplus workgroups exit) give
    the same bits as exact caps."""
    fmt, D, I, T, E, k = 4, 512, 256, 40, 64, 8
    from mvllm_hip import ACT_CLAMP_SWIGLU
    rng, pool, stride, geom, X, choice, mix, table = layer(hip, fmt, D, I, T, E, k, 5)
    a = run_routed(hip, fmt, D, I, table, route(hip, choice, mix, k), X, T, ACT_CLAMP_SWIGLU,
                   7.0, 0.0)[0]
    b = run_routed(hip, fmt, D, I, table, route(hip, choice, mix, k, cap_rows=T * k + 200,
                                                cap_e=E + 50), X, T, ACT_CLAMP_SWIGLU, 7.0,
                   0.0)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("fmt,ordered,mode", [(7, 0, 0), (7, 1, 0), (4, 0, 0), (4, 1, 1),
                                              (7, 0, 2)])
def test_routed_decode_split_rows_and_dead_rows(hip, orc, fmt, ordered, mode):
    """Hand-made segments on the decode path (S = 4 out rows): segments of 6 and 9 rows
    (more than S: split into items of S rows), rows whose out row is -1 or S (skipped), a
    repeated out row within a segment, and an out-of-table expert; against the oracle's
    moe_block on the same segments, with the folded and the ordered combine and each
    activation arithmetic (mode 0: two bf16 terms, bar 2e-5; mode 1: three, exact
    products, 2e-5; mode 2: one, the bf16 bar 1e-2)."""
    from mvllm_hip import ACT_CLAMP_SWIGLU, ACT_SITU, synth
    D, I, S, E = 512, 512, 4, 16
    act, a, b = (ACT_CLAMP_SWIGLU, 7.0, 0.0) if fmt == 4 else (ACT_SITU, 4.0, 25.0)
    rng, pool, stride, geom, X, _, _, table = layer(hip, fmt, D, I, S, E, 2, 404 + fmt)
    eids = np.array([3, 7, 40, 11], np.int32)   # 40: outside the table
    nr = np.array([6, 9, 2, 3], np.int32)
    xoff = np.concatenate([[0], np.cumsum(nr)[:-1]]).astype(np.int32)
    n = int(nr.sum())
    rows = rng.integers(0, S, n).astype(np.int32)
    rows[2], rows[8], rows[15] = -1, S, -3   # dead rows
    rows[9] = rows[10]                       # one out row twice in a segment
    rw = rng.uniform(0.1, 1.0, n).astype(np.float32)
    i32 = dict(dtype=torch.int32, device="cuda")
    seg = (torch.tensor([len(eids), n], **i32), dev(eids), dev(xoff), dev(nr), dev(rows),
           dev(rw))
    set_options(hip, combine_ordered=ordered, mode=mode)
    try:
        got, status = run_routed(hip, fmt, D, I, table, seg, X, S, act, a, b)
    finally:
        set_options(hip, combine_ordered=0, mode=0)
    assert status == 0
    lists = [[], [], [], [], [], []]
    for e in eids:
        pieces = synth.blob_pieces(pool[int(e)].cpu().numpy(), fmt, D, I, geom[1]) \
            if e < E else [None] * 6
        for j in range(6):
            lists[j].append(pieces[j])
    xg = X[np.clip(rows, 0, S - 1)]
    exp = np.zeros((S, D), np.float32)
    assert orc.moe_block(len(eids), D, I, fmt, *lists, xg, xoff, nr, rows, rw, exp, S,
                         act, a, b) == 1
    err = npref.rel_err(got, exp)
    say(f"split / dead rows (fmt={fmt}, ordered={ordered}, mode={mode}): rel_err", err)
    assert err < (1e-2 if mode == 2 else 2e-5)


def test_routed_decode_surplus_caps(hip):
    """Decode path: caps above the routed sizes (grids sized for them, surplus workgroups
    exit at the planner's item count) give the same bits as exact caps (ordered combine)."""
    fmt, D, I, T, E, k = 7, 1024, 512, 8, 64, 8
    from mvllm_hip import ACT_SITU
    rng, pool, stride, geom, X, choice, mix, table = layer(hip, fmt, D, I, T, E, k, 6)
    set_options(hip, combine_ordered=1, dec_ks=2)
    try:
        a = run_routed(hip, fmt, D, I, table, route(hip, choice, mix, k), X, T, ACT_SITU, 4.0,
                       25.0)[0]
        b = run_routed(hip, fmt, D, I, table, route(hip, choice, mix, k, cap_rows=T * k + 200,
                                                    cap_e=E + 50), X, T, ACT_SITU, 4.0, 25.0)[0]
    finally:
        set_options(hip, combine_ordered=0, dec_ks=0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _fp4_bar(got, exp):
    """Native-FP4 arithmetic against the composed oracle: exact e2m1 products, sums in
    another order, so an h value may land across an e2m1 rounding boundary now and then
    (the bar of the host-planned native-FP4 tests)."""
    den = np.max(np.abs(exp))
    rel = np.abs(got.astype(np.float64) - exp) / den
    say("  rel_err max", float(rel.max()), "p99", float(np.quantile(rel, 0.99)))
    assert float(rel.max()) < 1e-2
    assert float(np.quantile(rel, 0.99)) < 1e-5


def _oracle_fp4(orc, fmt, D, I, pool, geom, info, X, T, act, a, b, gone=()):
    from mvllm_hip import synth
    nb, eids, xoff, nr, rows, rw = info
    lists = [[], [], [], [], [], []]
    for e in eids:
        pieces = synth.blob_pieces(pool[int(e)].cpu().numpy(), fmt, D, I, geom[1]) \
            if int(e) not in gone else [None] * 6
        for j in range(6):
            lists[j].append(pieces[j])
    exp = np.zeros((T, D), np.float32)
    xg = X[np.clip(rows, 0, T - 1)]
    assert orc.moe_block_fp4act(nb, D, I, fmt, *lists, xg, xoff, nr, rows, rw, exp, T, act,
                                a, b) == 1
    return exp


@pytest.mark.parametrize("T,E,k,routing", [(6, 48, 4, "uniform"), (300, 64, 8, "skewed"),
                                           (700, 32, 4, "skewed")])
def test_routed_block_fp4act(hip, orc, T, E, k, routing):
    """Option fp4act on the device-resident block: every call size takes the native-MXFP4
    grouped path as the host-planned call does (x and H quantized to MXFP4, the scaled-FP4
    GEMM for blocks of 33-256 rows, bf16 copies of the quantized values for the 16- and
    32-row classes).  Bit for bit against the host-planned call on the same segments, and
    within the native-FP4 bar of the composed oracle (orc_moe_block_fp4act)."""
    from mvllm_hip import ACT_SITU
    fmt, D, I = 7, 1024, 512
    say("routed block fp4act", T, E, k, routing)
    rng, pool, stride, geom, X, choice, mix, table = layer(hip, fmt, D, I, T, E, k, 31 + T,
                                                          routing=routing)
    seg = route(hip, choice, mix, k)
    set_options(hip, fp4act=1)
    try:
        got, status = run_routed(hip, fmt, D, I, table, seg, X, T, ACT_SITU, 4.0, 25.0)
        ref, info = host_planned(hip, fmt, D, I, pool, stride, geom, seg, X, T, ACT_SITU, 4.0,
                                 25.0, table)
    finally:
        set_options(hip, fp4act=0)
    assert status == 0
    say(f"  segments {info[0]}, rows {int(info[3].sum())}, largest {int(info[3].max())}")
    if routing == "skewed":
        assert int(info[3].max()) > 64  # the scaled-FP4 classes run
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    _fp4_bar(got, _oracle_fp4(orc, fmt, D, I, pool, geom, info, X, T, ACT_SITU, 4.0, 25.0))


def test_routed_block_fp4act_dead_rows(hip, orc):
    """Hand-made segments under fp4act: rows whose out row is out of range (quantized as
    zero rows, never combined), a null expert and one outside the table (their rows
    consumed without writing), a segment of 300 rows (a full 256-row block and a
    remainder); caps above the sizes."""
    from mvllm_hip import ACT_SITU
    fmt, D, I, S, E = 7, 512, 256, 24, 16
    rng, pool, stride, geom, X, _, _, table = layer(hip, fmt, D, I, S, E, 2, 808,
                                                    null_ids=(5,))
    eids = np.array([3, 5, 40, 11, 2], np.int32)  # 5: null; 40: outside the table
    nr = np.array([300, 20, 7, 40, 3], np.int32)
    xoff = np.concatenate([[0], np.cumsum(nr)[:-1]]).astype(np.int32)
    n = int(nr.sum())
    rows = rng.integers(0, S, n).astype(np.int32)
    rows[[2, 50, 333, 360]] = [-1, S, -7, S + 3]
    rw = rng.uniform(0.1, 1.0, n).astype(np.float32)
    i32 = dict(dtype=torch.int32, device="cuda")
    pad = 64  # caps above the sizes
    seg = (torch.tensor([len(eids), n], **i32),
           dev(np.concatenate([eids, np.zeros(pad, np.int32)])),
           dev(np.concatenate([xoff, np.zeros(pad, np.int32)])),
           dev(np.concatenate([nr, np.zeros(pad, np.int32)])),
           dev(np.concatenate([rows, np.zeros(pad, np.int32)])),
           dev(np.concatenate([rw, np.zeros(pad, np.float32)])))
    set_options(hip, fp4act=1)
    try:
        got, status = run_routed(hip, fmt, D, I, table, seg, X, S, ACT_SITU, 4.0, 25.0)
    finally:
        set_options(hip, fp4act=0)
    assert status == 0
    info = (len(eids), eids, xoff, nr, rows, rw)
    exp = _oracle_fp4(orc, fmt, D, I, pool, geom, info, X, S, ACT_SITU, 4.0, 25.0,
                      gone=(5, 40))
    _fp4_bar(got, exp)


@pytest.mark.parametrize("fmt,E", [(7, 256), (4, 160)])
def test_routed_decode_self_planned(hip, orc, fmt, E):
    """The default decode path, whose gate/up kernel finds its own item among the segments
    (64 segments per scan step): a call of 16 tokens over more than 64 routed experts (two
    or more scan steps), against the ordered path (the planner kernel's descriptors) within
    the float-atomic combine's bar, against the oracle chain, and with caps above the
    routed sizes (surplus workgroups find no item)."""
    from mvllm_hip import ACT_CLAMP_SWIGLU, ACT_SITU
    D, I, T, k = 1024, 512, 16, 8
    act, a, b = (ACT_CLAMP_SWIGLU, 7.0, 0.0) if fmt == 4 else (ACT_SITU, 4.0, 25.0)
    rng, pool, stride, geom, X, choice, mix, table = layer(hip, fmt, D, I, T, E, k, 61 + E)
    seg = route(hip, choice, mix, k)
    nb = int(seg[0].cpu().numpy()[0])
    say(f"self-planned decode: fmt {fmt}, {nb} segments")
    assert nb > 64
    got, status = run_routed(hip, fmt, D, I, table, seg, X, T, act, a, b)
    assert status == 0
    set_options(hip, combine_ordered=1)
    try:
        ordered, status = run_routed(hip, fmt, D, I, table, seg, X, T, act, a, b)
    finally:
        set_options(hip, combine_ordered=0)
    assert status == 0
    say("  vs ordered: rel", npref.rel_err(got, ordered))
    assert npref.rel_err(got, ordered) < 1e-5
    exp = oracle_chain(orc, fmt, D, I, pool, stride, geom, choice, mix, k, X, T, act, a, b)
    say("  vs oracle chain: rel", npref.rel_err(got, exp))
    assert npref.rel_err(got, exp) < 2e-5
    big = route(hip, choice, mix, k, cap_rows=T * k + 300, cap_e=E + 40)
    got2, status = run_routed(hip, fmt, D, I, table, big, X, T, act, a, b)
    assert status == 0
    say("  surplus caps vs exact: rel", npref.rel_err(got2, got))
    assert npref.rel_err(got2, got) < 1e-6
