"""Golden fixtures written by the reference's own moe_block (tests/golden/make_golden.py):
the oracle reproduces them bit for bit on CPU, and the HIP path stays within the decode
tolerance of them on the GPU.  The inputs are regenerated from seeds; a digest stored with
each fixture proves they are the inputs the reference saw."""
import os

import numpy as np
import pytest

import npref

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def _load():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden",
                                                  os.path.join(GOLDEN, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


MG = _load()
NAMES = sorted(MG.FIXTURES)


def _fixture(name):
    kind, p = MG.FIXTURES[name]
    args, act, a, b, flat = MG.build_inputs(kind, p)
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    assert str(z["digest"]) == MG.digest(flat), "regenerated inputs differ from the fixture's"
    return args, act, a, b, z["out"]


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_golden(orc, name):
    args, act, a, b, gold = _fixture(name)
    out = args[15].copy()
    assert orc.moe_block(*args[:15], out, args[16], act, a, b) == 1
    assert np.array_equal(out.view(np.uint32), gold.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_matches_golden(hip, name):
    import torch
    args, act, a, b, gold = _fixture(name)
    keep = []

    def dl(xs):
        if xs is None:
            return None
        r = []
        for x in xs:
            if x is None:
                r.append(None)
                continue
            t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
            keep.append(t)
            r.append(t.data_ptr())
        return r
    nb, D, I, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out0, S = args
    xg_d = torch.from_numpy(np.ascontiguousarray(xg)).cuda()
    out_d = torch.from_numpy(out0.copy()).cuda()
    hip.moe_block_dev(nb, D, I, fmt, dl(g), dl(u), dl(d), dl(gs), dl(us), dl(ds), xg_d, xoff, nr,
                      rows, rw, out_d, S, act, a, b)
    torch.cuda.synchronize()
    got = out_d.cpu().numpy()
    err = npref.rel_err(got, gold)
    print(name, "rel_err", err, flush=True)
    assert err < 2e-5
