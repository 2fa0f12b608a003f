"""mvllm_hip_moe_block_dev_noalloc (the entry that allocates no device memory) against
mvllm_hip_moe_block_dev, through the C ABI: the same results on two calls in a row, the
second with a smaller input, on the decode kernels and on the grouped GEMM; a call past
the scratch limit is refused with a message, and the entry works again after it."""
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
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def lists(c, keep):
    def L(xs):
        if xs is None:
            return None
        out = []
        for x in xs:
            t = None if x is None else dev(x)
            keep.append(t)
            out.append(None if t is None else t.data_ptr())
        return out
    return [L(c.g), L(c.u), L(c.d), L(c.gs), L(c.us), L(c.ds)]


def both(hip, c):
    """(moe_block_dev result, moe_block_dev_noalloc result) of the same call."""
    keep = []
    ls = lists(c, keep)
    xg = dev(c.xg)
    o1, o2 = dev(c.out), dev(c.out)
    hip.moe_block_dev(c.nb, c.D, c.I, c.fmt, *ls, xg, c.xoff, c.nr, c.rows, c.rw, o1, c.S,
                      c.act, c.a, c.b)
    hip.moe_block_dev_noalloc(c.nb, c.D, c.I, c.fmt, *ls, xg, c.xoff, c.nr, c.rows, c.rw, o2,
                              c.S, c.act, c.a, c.b)
    torch.cuda.synchronize()
    return o1.cpu().numpy(), o2.cpu().numpy()


# (fmt, D, I, nr, S, act, a, b): a larger call, then a smaller one
PAIRS = [
    ("decode", (4, 2048, 1024, [1] * 8, 4, 0, 0.0, 0.0), (4, 2048, 1024, [2, 1, 1], 3, 0, 0.0, 0.0)),
    ("decode-mxfp4", (7, 7168, 2048, [1] * 8, 1, 2, 4.0, 25.0), (7, 7168, 2048, [1, 1], 1, 2, 4.0, 25.0)),
    ("gemm", (4, 1024, 512, [40, 17, 3, 70], 64, 1, 7.0, 0.0), (4, 1024, 512, [20, 5], 16, 1, 7.0, 0.0)),
    ("gemm-mxfp4", (7, 1024, 512, [200, 5, 33], 128, 2, 4.0, 25.0), (7, 512, 256, [18], 8, 2, 4.0, 25.0)),
    ("exact", (4, 96, 70, [2, 1], 3, 1, 0.0, 0.0), (4, 77, 33, [1], 1, 0, 0.0, 0.0)),
]


@pytest.mark.parametrize("name,big,small", PAIRS, ids=[p[0] for p in PAIRS])
@pytest.mark.parametrize("ordered", [1, 0])
def test_noalloc_matches_dev(hip, name, big, small, ordered):
    """Ordered combine: bit-identical to moe_block_dev (same kernels, same plan, buffers in
    the scratch array).  Default (decode calls fold the combine with float atomics): within
    the decode bar of the oracle-pinned entry."""
    assert hip.set_option("combine_ordered", ordered)
    try:
        for k, (fmt, D, I, nr, S, act, a, b) in enumerate((big, small)):
            say("noalloc", name, "ordered" if ordered else "atomic", "call", k, nr)
            rng = np.random.default_rng(1000 + 17 * k + D + I + fmt)
            c = random_case(rng, fmt, D, I, nr, S, act, a, b)
            r1, r2 = both(hip, c)
            if ordered or name.startswith("gemm") or name == "exact":
                assert np.array_equal(r1.view(np.uint32), r2.view(np.uint32))
            else:
                assert npref.rel_err(r2, r1) < TOL_F32
    finally:
        hip.set_option("combine_ordered", 0)


def test_noalloc_refuses_oversize_then_runs(hip):
    """A call whose buffers exceed the scratch array returns 0 with a message and enqueues
    nothing; the next call that fits runs and matches moe_block_dev."""
    say("noalloc oversize")
    D, I, n = 2048, 1024, 4000   # grouped GEMM: 4000 * (2D + 2I + 4D) bytes > 47.75 MiB
    keep = []
    w = [torch.zeros((I, D // 2), dtype=torch.uint8, device="cuda") for _ in range(3)]
    s = [torch.ones((I, D // 64), dtype=torch.float32, device="cuda") for _ in range(3)]
    keep += w + s
    p = lambda ts: [t.data_ptr() for t in ts]
    xg = torch.zeros((n, D), dtype=torch.float32, device="cuda")
    out = torch.zeros((n, D), dtype=torch.float32, device="cuda")
    rows = np.arange(n, dtype=np.int32)
    rw = np.ones(n, np.float32)
    rc = hip.moe_block_dev_noalloc(1, D, I, 4, p(w[:1]), p(w[1:2]), p(w[2:]), p(s[:1]), p(s[1:2]),
                                   p(s[2:]), xg, np.zeros(1, np.int32), np.array([n], np.int32),
                                   rows, rw, out, n, 0, 0.0, 0.0, check=False)
    assert rc == 0
    msg = hip.lib().mvllm_hip_last_error().decode()
    say("  refused:", msg)
    assert "scratch" in msg
    torch.cuda.synchronize()
    assert float(out.abs().max()) == 0.0
    rng = np.random.default_rng(5)
    c = random_case(rng, 4, 1024, 512, [3, 1, 2], 4, 1, 7.0, 0.0)
    assert hip.set_option("combine_ordered", 1)
    try:
        r1, r2 = both(hip, c)
    finally:
        hip.set_option("combine_ordered", 0)
    assert np.array_equal(r1.view(np.uint32), r2.view(np.uint32))
