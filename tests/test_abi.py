"""CPU checks of the C-ABI library: it loads, exports every symbol the public header
declares, and its host-side integer work (segments, union, blob geometry) is
bit-exact with the oracle.  No compute is run (there is no GPU here)."""
import ctypes

import numpy as np
import pytest

import mvllm_hip


def test_library_exports_header_symbols():
    L = mvllm_hip.lib()
    syms = mvllm_hip.header_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    assert mvllm_hip.lib().mvllm_hip_name() == b"hip"


def test_not_initialised_falls_back():
    # before init every compute entry returns 0 ("use the host kernel")
    L = mvllm_hip.lib()
    if L.mvllm_hip_available():
        pytest.skip("already initialised in this process")
    x = np.zeros((1, 64), np.float32)
    out = np.zeros((1, 64), np.float32)
    one = np.array([1], np.int32)
    zero = np.array([0], np.int32)
    rc = mvllm_hip.moe_block(1, 64, 64, 4, None, None, None, None, None, None, x, zero, one,
                             zero, np.ones(1, np.float32), out, 1, check=False)
    assert rc == 0
    assert b"init" in L.mvllm_hip_last_error()


@pytest.mark.parametrize("seed,T,E,k", [(1, 1, 8, 2), (2, 16, 64, 8), (3, 97, 33, 5),
                                        (4, 512, 256, 8)])
def test_segments_bit_exact_vs_oracle(orc, seed, T, E, k):
    rng = np.random.default_rng(seed)
    idx = rng.integers(-1, E, size=(T, k)).astype(np.int32)
    wt = rng.uniform(0, 1, size=(T, k)).astype(np.float32)
    wt[rng.random((T, k)) < 0.05] = 0.0
    a = mvllm_hip.segments(idx, wt, T, k, E)
    b = orc.moe_segments(idx, wt, T, k, E)
    assert a[0] == b[0]
    for x, y in zip(a[1:], b[1:]):
        assert np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32))
    assert np.array_equal(mvllm_hip.union_ids(idx, T, k, E), orc.moe_union_ids(idx, T, k, E))


def test_segments_cancelling_weights():
    # wsum == 0 drops the row even when the slot weights are non-zero (+w, -w)
    idx = np.array([[3, 3, 1]], np.int32)
    wt = np.array([[0.25, -0.25, 0.5]], np.float32)
    nb, eids, xoff, nr, rows, rw = mvllm_hip.segments(idx, wt, 1, 3, 8)
    assert list(eids) == [1, 3] and list(nr) == [1, 0] and list(rows) == [0]


@pytest.mark.parametrize("fmt,D,I", [(4, 1024, 512), (4, 6144, 2048), (4, 100, 70),
                                     (7, 7168, 2048), (7, 96, 33)])
def test_expert_geom(fmt, D, I):
    n, off = mvllm_hip.expert_geom(fmt, D, I)
    gq, sb = (64, 4) if fmt == 4 else (32, 1)
    pg, sg = I * ((D + 1) // 2), I * ((D + gq - 1) // gq) * sb
    pd, sd = D * ((I + 1) // 2), D * ((I + gq - 1) // gq) * sb
    assert n == 2 * (pg + sg) + pd + sd
    if fmt == 4:  # gate_p | gate_s | up_p | up_s | down_p | down_s
        assert list(off) == [0, pg, pg + sg, 2 * pg + sg, 2 * (pg + sg), 2 * (pg + sg) + pd]
    else:  # w1p | w1s | w2p | w2s | w3p | w3s, gate=w1 down=w2 up=w3
        assert list(off) == [0, pg, pg + sg + pd + sd, 2 * pg + sg + pd + sd, pg + sg,
                             pg + sg + pd]
    assert mvllm_hip.expert_geom(5, D, I)[0] == -1
