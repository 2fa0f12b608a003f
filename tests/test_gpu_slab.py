"""Expert containers into HBM (mvllm_hip_slab_load): every blob of the slab holds the
bytes the container wrote for that (layer, expert) in the blob layout, the device table
holds the blob addresses, and moe_block on the slab's pointers matches the oracle on the
container's bytes (src/model/glm53.cpp:1829-1871, src/model/kimi_k3.cpp:1881-1934)."""
import ctypes
import sys

import numpy as np
import pytest
import torch

import npref
from st_fixture import make_container

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def d2h(addr, nbytes):
    """Device bytes at a raw address, through the HIP runtime torch has loaded."""
    rt = ctypes.CDLL("libamdhip64.so.7")
    out = np.empty(nbytes, np.uint8)
    torch.cuda.synchronize()
    rc = rt.hipMemcpy(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(addr),
                      ctypes.c_size_t(nbytes), 2)  # hipMemcpyDeviceToHost
    assert rc == 0
    return out


@pytest.mark.parametrize("fmt,D,I,n_files", [(7, 512, 256, 2), (4, 512, 256, 3)])
def test_slab_holds_the_container(hip, orc, tmp_path, fmt, D, I, n_files):
    say("slab", fmt, D, I, n_files)
    rng = np.random.default_rng(fmt + n_files)
    prefix = "model." if fmt == 4 else ""
    layers, E = [1, 2, 3], 5
    blobs = make_container(str(tmp_path), rng, fmt, D, I, layers, E, prefix, n_files=n_files)
    slab = hip.Slab(str(tmp_path), prefix, fmt, D, I, 2, 4, E)
    try:
        assert slab.n_blobs == 2 * E and slab.stride % 256 == 0
        assert slab.blob_bytes == len(blobs[(2, 0)])
        for L in (2, 3):
            for e in range(E):
                got = d2h(slab.blob(L, e), slab.blob_bytes).tobytes()
                assert got == blobs[(L, e)], (L, e)
        table = d2h(slab.table, 8 * slab.n_blobs).view(np.uint64)
        assert table.tolist() == [slab.blob(L, e) for L in (2, 3) for e in range(E)]
        # moe_block on three of layer 3's experts straight from the slab
        geom = hip.expert_geom(fmt, D, I)
        off = geom[1]
        order = (0, 2, 4, 1, 3, 5)  # gate_p gate_s up_p up_s down_p down_s -> g u d gs us ds
        eids = [4, 0, 2]
        nr = np.array([3, 1, 2], np.int32)
        ptrs = [[slab.blob(3, e) + int(off[o]) for e in eids] for o in order]
        R, S = int(nr.sum()), 4
        x = rng.standard_normal((R, D)).astype(np.float32)
        xoff = np.array([0, 3, 4], np.int32)
        rows = rng.integers(0, S, R).astype(np.int32)
        rw = rng.uniform(0.1, 1.0, R).astype(np.float32)
        act, a, b = (1, 7.0, 0.0) if fmt == 4 else (2, 4.0, 25.0)
        out = torch.zeros((S, D), dtype=torch.float32, device="cuda")
        hip.moe_block_dev(3, D, I, fmt, *ptrs, torch.from_numpy(x).cuda(), xoff, nr, rows, rw,
                          out, S, act, a, b)
        torch.cuda.synchronize()
        pieces = []
        for e in eids:
            raw = np.frombuffer(blobs[(3, e)], np.uint8)
            pieces.append([raw[int(off[o]):] for o in order])
        lists = []
        for j in range(6):
            L = []
            for p in pieces:
                seg = p[j]
                if j >= 3 and fmt == 4:
                    seg = seg[:(len(seg) // 4) * 4].view(np.float32)
                L.append(np.ascontiguousarray(seg))
            lists.append(L)
        exp = np.zeros((S, D), np.float32)
        assert orc.moe_block(3, D, I, fmt, *lists, x, xoff, nr, rows, rw, exp, S, act, a, b) == 1
        err = npref.rel_err(out.cpu().numpy(), exp)
        say("  moe_block from the slab: rel_err", err)
        assert err < 2e-5
    finally:
        slab.free()


def test_slab_errors(hip, tmp_path):
    rng = np.random.default_rng(9)
    make_container(str(tmp_path), rng, 7, 256, 128, [1], 2, "")
    with pytest.raises(hip.HipError, match="wrong size at L1 E0"):
        hip.Slab(str(tmp_path), "", 7, 256, 256, 1, 2, 2)
    with pytest.raises(hip.HipError, match="missing or wrong size at L1 E2"):
        hip.Slab(str(tmp_path), "", 7, 256, 128, 1, 2, 3)
    assert hip.lib().mvllm_hip_slab_free(12345) == 0
