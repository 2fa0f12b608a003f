"""Python binding of libmvllm_hip.so (the C ABI in include/mvllm_hip.h).

The library is the product; this module only marshals arguments for tests and
bench.py.  It never falls back to a CPU implementation: if the shared library is
missing or the device is absent, calls raise.

torch is imported before the library is loaded when it is installed: torch ships
its own libamdhip64.so (SONAME libamdhip64.so.7), and loading ours first would put
a second HIP runtime into the process.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

try:  # must precede CDLL (one HIP runtime per process)
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of this image
    torch = None

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libmvllm_hip.so")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "mvllm_hip.h")

ACT_SILU, ACT_CLAMP_SWIGLU, ACT_SITU = 0, 1, 2
STAT_NAMES = ["calls", "rows", "h2d_weight_bytes", "h2d_act_bytes", "d2h_bytes", "promotions",
              "resident_hits", "misses", "evictions", "ms_gate_up", "ms_down", "ms_combine",
              "ms_prep", "launches_gate_up", "launches_down", "host_ms", "host_wait_ms",
              "tier_bytes", "tier_parked_bytes", "host_plan_ms"]

_i, _f, _p, _sz, _ll = C.c_int, C.c_float, C.c_void_p, C.c_size_t, C.c_longlong
_pp = C.POINTER(C.c_void_p)

_SIGS = {
    "mvllm_hip_init": (_i, [_i]),
    "mvllm_hip_shutdown": (None, []),
    "mvllm_hip_available": (_i, []),
    "mvllm_hip_name": (C.c_char_p, []),
    "mvllm_hip_last_error": (C.c_char_p, []),
    "mvllm_hip_moe_block": (_i, [_i, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _pp, _p, _p, _p, _p,
                                 _p, _p, _i, _i, _f, _f]),
    "mvllm_hip_moe_block_dev": (_i, [_i, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _pp, _p, _p,
                                     _p, _p, _p, _p, _i, _i, _f, _f, _p]),
    "mvllm_hip_moe_block_dev_noalloc": (_i, [_i, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _pp,
                                             _p, _p, _p, _p, _p, _p, _i, _i, _f, _f, _p]),
    "mvllm_hip_set_option": (_i, [C.c_char_p, _ll]),
    "mvllm_moe_union_ids": (_i, [_p, _i, _i, _p, _i]),
    "mvllm_moe_segments": (_i, [_p, _p, _i, _i, _p, _p, _p, _p, _p, _i, _i, _p]),
    "mvllm_expert_geom": (_ll, [_i, _i, _i, _p]),
    "mvllm_hip_host_alloc": (_p, [_sz]),
    "mvllm_hip_host_free": (_i, [_p]),
    "mvllm_hip_set_expert_budget": (_i, [_sz]),
    "mvllm_hip_promote": (_i, [_p, _sz, _i, _i]),
    "mvllm_hip_evict": (_i, [_i, _i]),
    "mvllm_hip_resident_ptr": (_p, [_i, _i]),
    "mvllm_hip_stats": (_i, [_p, _i]),
    "mvllm_hip_stats_reset": (None, []),
    "mvllm_hip_dequant": (_i, [_i, _p, _p, _i, _i, _p]),
    "mvllm_hip_quantize_mxfp4": (_i, [_p, _i, _i, _p, _p, _p]),
    "mvllm_hip_bf16_planes": (_i, [_i, _i, _p, _i, _i, _p]),
    "mvllm_hip_router_dev": (_i, [_p, _p, _p, _i, _i, _i, _i, _f, _p, _p, _p, _p, _p]),
    "mvllm_hip_linear_dev": (_i, [_i, _p, _p, _i, _i, _p, _i, _p, _p]),
    "mvllm_hip_rmsnorm_dev": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "mvllm_hip_moe_topk_dev": (_i, [_p, _p, _i, _i, _i, _p, _p, _p]),
    "mvllm_hip_moe_segments_dev": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _i, _p,
                                        _p]),
    "mvllm_hip_moe_route_dev": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i,
                                     _p, _p]),
    "mvllm_hip_membench": (_i, [_i, _p, _p, _sz, _i, _i, _p]),
    "mvllm_st_expert_pieces": (_i, [C.c_char_p, C.c_char_p, _i, _i, _i, _i, _i, _i, _p, _p, _p,
                                    _p, _ll, _p, _ll]),
    "mvllm_hip_slab_load": (_ll, [C.c_char_p, C.c_char_p, _i, _i, _i, _i, _i, _i]),
    "mvllm_hip_slab_info": (_i, [_ll, _pp, _pp, _p, _p, _p]),
    "mvllm_hip_slab_free": (_i, [_ll]),
    "mvllm_hip_prefetch": (_i, [_i, _p, _p, _pp, _p]),
    "mvllm_hip_repin": (_i, [_i, _p]),
    "mvllm_hip_host_reuse": (_i, [_p, _sz]),
    "mvllm_hip_tier_table": (_i, [_i, _i, _p, _p, _p]),
    "mvllm_hip_tier_table_done": (_i, [_i, _p]),
    "mvllm_hip_moe_block_routed_dev": (_i, [_i, _i, _i, _p, _i, _p, _p, _p, _p, _i, _p, _p, _i,
                                            _p, _p, _i, _i, _f, _f, _p, _p]),
}

_lib = None


def lib():
    """Load libmvllm_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def header_symbols():
    """Every function name the public header declares."""
    import re
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mvllm_[a-z0-9_]+)\s*\(", text)))


class HipError(RuntimeError):
    pass


def _check(rc, what):
    if rc != 1:
        raise HipError(f"{what} failed: {lib().mvllm_hip_last_error().decode()}")


def init(device: int = 0):
    _check(lib().mvllm_hip_init(device), "mvllm_hip_init")


def shutdown():
    lib().mvllm_hip_shutdown()


def set_option(key: str, value: int) -> bool:
    return lib().mvllm_hip_set_option(key.encode(), int(value)) == 1


def _ptr(a):
    if a is None or isinstance(a, int):  # an address the caller already holds
        return a
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()  # torch tensor


def _ptr_array(items):
    arr = (C.c_void_p * len(items))()
    for i, a in enumerate(items):
        arr[i] = None if a is None else (a if isinstance(a, int) else _ptr(a))
    return arr


def moe_block(nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S,
              act=ACT_SILU, act_a=0.0, act_b=0.0, qgs=0, check=True):
    """Host-pointer drop-in (numpy arrays).  Lists may hold None; any list may be None."""
    pa = [None if L is None else _ptr_array(L) for L in (g, u, d, gs, us, ds)]
    rc = lib().mvllm_hip_moe_block(nb, D, Iinter, fmt, qgs, *pa, _ptr(xg), _ptr(xoff), _ptr(nr),
                                   _ptr(rows), _ptr(rw), _ptr(out), S, act, act_a, act_b)
    if check:
        _check(rc, "mvllm_hip_moe_block")
    return rc


def prepare_lists(g, u, d, gs, us, ds):
    """Pointer lists -> ctypes arrays, reusable across moe_block_dev calls."""
    return tuple(None if L is None else _ptr_array(L) for L in (g, u, d, gs, us, ds))


def moe_block_dev(nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S,
                  act=ACT_SILU, act_a=0.0, act_b=0.0, stream=None, check=True, prepared=None):
    """Device variant: g..ds are lists of device pointers (ints) or torch tensors;
    xg/out are torch CUDA tensors; xoff/nr/rows/rw are numpy host arrays.  Any of the
    arrays may also be given as its address (int), which saves the per-call lookup.
    `prepared` (from prepare_lists) replaces g..ds when given."""
    pa = prepared if prepared is not None else \
        [None if L is None else _ptr_array(L) for L in (g, u, d, gs, us, ds)]
    st = None if stream is None else (stream if isinstance(stream, int) else stream.cuda_stream)
    rc = lib().mvllm_hip_moe_block_dev(nb, D, Iinter, fmt, 0, *pa, _ptr(xg), _ptr(xoff),
                                       _ptr(nr), _ptr(rows), _ptr(rw), _ptr(out), S, act, act_a,
                                       act_b, st)
    if check:
        _check(rc, "mvllm_hip_moe_block_dev")
    return rc


def moe_block_dev_noalloc(nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out,
                          S, act=ACT_SILU, act_a=0.0, act_b=0.0, stream=None, check=True,
                          prepared=None):
    """mvllm_hip_moe_block_dev_noalloc: moe_block_dev's arguments, no device allocation."""
    pa = prepared if prepared is not None else \
        [None if L is None else _ptr_array(L) for L in (g, u, d, gs, us, ds)]
    st = None if stream is None else (stream if isinstance(stream, int) else stream.cuda_stream)
    rc = lib().mvllm_hip_moe_block_dev_noalloc(nb, D, Iinter, fmt, 0, *pa, _ptr(xg), _ptr(xoff),
                                               _ptr(nr), _ptr(rows), _ptr(rw), _ptr(out), S, act,
                                               act_a, act_b, st)
    if check:
        _check(rc, "mvllm_hip_moe_block_dev_noalloc")
    return rc


def union_ids(idx, n_tok, topk, cap):
    idx = np.ascontiguousarray(idx, np.int32)
    out = np.full(max(cap, 1), -7, np.int32)
    n = lib().mvllm_moe_union_ids(_ptr(idx), n_tok, topk, _ptr(out), cap)
    return out[:n]


def segments(idx, wt, n_tok, topk, cap_experts):
    """-> (nb, eids, xoff, nr, rows, rw) for one batched moe_block call."""
    idx = np.ascontiguousarray(idx, np.int32)
    wt = np.ascontiguousarray(wt, np.float32)
    cap_rows = max(n_tok * topk, 1)
    eids = np.zeros(cap_experts, np.int32)
    xoff = np.zeros(cap_experts, np.int32)
    nr = np.zeros(cap_experts, np.int32)
    rows = np.zeros(cap_rows, np.int32)
    rw = np.zeros(cap_rows, np.float32)
    nrows = np.zeros(1, np.int32)
    nb = lib().mvllm_moe_segments(_ptr(idx), _ptr(wt), n_tok, topk, _ptr(eids), _ptr(xoff),
                                  _ptr(nr), _ptr(rows), _ptr(rw), cap_experts, cap_rows,
                                  _ptr(nrows))
    if nb < 0:
        raise HipError("mvllm_moe_segments: capacity too small")
    j = int(nrows[0])
    return nb, eids[:nb], xoff[:nb], nr[:nb], rows[:j], rw[:j]


def expert_geom(fmt, D, Iinter):
    """-> (blob_bytes, offsets[6] = gate_p, gate_s, up_p, up_s, down_p, down_s)."""
    off = np.zeros(6, np.int64)
    n = lib().mvllm_expert_geom(fmt, D, Iinter, _ptr(off))
    return int(n), off


def promote(host_blob_ptr: int, nbytes: int, layer: int, eid: int):
    _check(lib().mvllm_hip_promote(host_blob_ptr, nbytes, layer, eid), "mvllm_hip_promote")


def evict(layer, eid) -> bool:
    return lib().mvllm_hip_evict(layer, eid) == 1


def stats():
    v = np.zeros(len(STAT_NAMES), np.float64)
    n = lib().mvllm_hip_stats(_ptr(v), len(v))
    return dict(zip(STAT_NAMES[:n], v[:n].tolist()))


def stats_reset():
    lib().mvllm_hip_stats_reset()


def dequant(fmt, packed_dev, scales_dev, O, K, w_dev):
    _check(lib().mvllm_hip_dequant(fmt, _ptr(packed_dev), _ptr(scales_dev), O, K, _ptr(w_dev)),
           "mvllm_hip_dequant")


def _stream(stream):
    return None if stream is None else (stream if isinstance(stream, int) else stream.cuda_stream)


def moe_topk_dev(choice, mix, n_tok, n_exp, k, idx, wt, stream=None):
    """moe_topk of every token on the device (see mvllm_hip_moe_topk_dev); enqueued."""
    _check(lib().mvllm_hip_moe_topk_dev(_ptr(choice), _ptr(mix), n_tok, n_exp, k, _ptr(idx),
                                        _ptr(wt), _stream(stream)), "mvllm_hip_moe_topk_dev")


def moe_segments_dev(idx, wt, n_tok, topk, n_exp, work, eids, xoff, nr, rows, rw, counts,
                     stream=None):
    """mvllm_moe_segments on the device (see mvllm_hip_moe_segments_dev); enqueued.
    Capacities are the lengths of eids and rows."""
    _check(lib().mvllm_hip_moe_segments_dev(_ptr(idx), _ptr(wt), n_tok, topk, n_exp, _ptr(work),
                                            _ptr(eids), _ptr(xoff), _ptr(nr), _ptr(rows),
                                            _ptr(rw), len(eids), len(rows), _ptr(counts),
                                            _stream(stream)), "mvllm_hip_moe_segments_dev")


def moe_route_dev(choice, mix, n_tok, n_exp, k, idx, wt, work, eids, xoff, nr, rows, rw,
                  counts, stream=None):
    """moe_topk_dev then moe_segments_dev in one call (see mvllm_hip_moe_route_dev)."""
    _check(lib().mvllm_hip_moe_route_dev(_ptr(choice), _ptr(mix), n_tok, n_exp, k, _ptr(idx),
                                         _ptr(wt), _ptr(work), _ptr(eids), _ptr(xoff), _ptr(nr),
                                         _ptr(rows), _ptr(rw), len(eids), len(rows), _ptr(counts),
                                         _stream(stream)), "mvllm_hip_moe_route_dev")


def moe_block_routed_dev(D, Iinter, fmt, table, n_table, counts, eids, xoff, nr, rows, rw, x,
                         out, S, act=ACT_SILU, act_a=0.0, act_b=0.0, status=None, stream=None):
    """mvllm_hip_moe_block_routed_dev: segments (counts, eids, xoff, nr, rows, rw) and the
    blob table in device memory; caps are the lengths of eids and rows.  Enqueued."""
    _check(lib().mvllm_hip_moe_block_routed_dev(D, Iinter, fmt, _ptr(table), n_table,
                                                _ptr(counts), _ptr(eids), _ptr(xoff), _ptr(nr),
                                                len(eids), _ptr(rows), _ptr(rw), len(rows),
                                                _ptr(x), _ptr(out), S, act, act_a, act_b,
                                                _ptr(status), _stream(stream)),
           "mvllm_hip_moe_block_routed_dev")


def router_dev(x, w, bias, n_tok, D, n_exp, k, rscale, scores, choice, idx, wt, stream=None):
    """cpu_route of every token row on the device (see mvllm_hip_router_dev); enqueued."""
    _check(lib().mvllm_hip_router_dev(_ptr(x), _ptr(w), _ptr(bias), n_tok, D, n_exp, k, rscale,
                                      _ptr(scores), _ptr(choice), _ptr(idx), _ptr(wt),
                                      _stream(stream)), "mvllm_hip_router_dev")


def linear_dev(fmt, w, scales, O, K, x, n, y, stream=None):
    """y[n, O] = x[n, K] . W^T on the device (see mvllm_hip_linear_dev); enqueued."""
    _check(lib().mvllm_hip_linear_dev(fmt, _ptr(w), _ptr(scales), O, K, _ptr(x), n, _ptr(y),
                                      _stream(stream)), "mvllm_hip_linear_dev")


def rmsnorm_dev(x, w, y, rows, n, eps, stream=None):
    _check(lib().mvllm_hip_rmsnorm_dev(_ptr(x), _ptr(w), _ptr(y), rows, n, eps,
                                       _stream(stream)), "mvllm_hip_rmsnorm_dev")


def bf16_planes(fmt, terms, x_dev, n, K, planes_dev):
    _check(lib().mvllm_hip_bf16_planes(fmt, terms, _ptr(x_dev), n, K, _ptr(planes_dev)),
           "mvllm_hip_bf16_planes")


def quantize_mxfp4(x_dev, n, K, codes_dev, scales_dev, planes_dev=None):
    """MXFP4 codes + ue8m0 scales of x [n, K]; planes_dev (optional, bf16/int16 [n, K]):
    the quantized values as bf16."""
    _check(lib().mvllm_hip_quantize_mxfp4(_ptr(x_dev), n, K, _ptr(codes_dev), _ptr(scales_dev),
                                          _ptr(planes_dev)),
           "mvllm_hip_quantize_mxfp4")


def membench(kind, src, dst, nbytes, row_bytes=0, reps=5):
    """-> ms per repetition of the memory probe (see mvllm_hip_membench)."""
    ms = np.zeros(1, np.float64)
    _check(lib().mvllm_hip_membench(kind, _ptr(src), _ptr(dst), nbytes, row_bytes, reps,
                                    _ptr(ms)), "mvllm_hip_membench")
    return float(ms[0])


def st_expert_pieces(dirpath, prefix, fmt, D, Iinter, layer0, layer1, n_experts):
    """-> (paths, file [n, 6], offset [n, 6], bytes [n, 6]) for n = (layer1 - layer0) *
    n_experts blobs; raises HipError with the reference's message when a piece is missing
    or has the wrong size (see mvllm_st_expert_pieces).  Host only."""
    n = (layer1 - layer0) * n_experts * 6
    fi = np.zeros(max(n, 1), np.int32)
    off = np.zeros(max(n, 1), np.int64)
    nb = np.zeros(max(n, 1), np.int64)
    paths = C.create_string_buffer(1 << 16)
    err = C.create_string_buffer(1024)
    r = lib().mvllm_st_expert_pieces(dirpath.encode(), (prefix or "").encode(), fmt, D, Iinter,
                                     layer0, layer1, n_experts, _ptr(fi), _ptr(off), _ptr(nb),
                                     C.cast(paths, C.c_void_p), len(paths),
                                     C.cast(err, C.c_void_p), len(err))
    if r < 0:
        raise HipError(err.value.decode())
    files = [p for p in paths.value.decode().split("\n") if p]
    return files, fi[:n].reshape(-1, 6), off[:n].reshape(-1, 6), nb[:n].reshape(-1, 6)


class Slab:
    """A layer range of routed experts read from safetensors containers into HBM (see
    mvllm_hip_slab_load).  .base / .table are device addresses, .stride the blob stride."""

    def __init__(self, dirpath, prefix, fmt, D, Iinter, layer0, layer1, n_experts):
        h = lib().mvllm_hip_slab_load(dirpath.encode(), (prefix or "").encode(), fmt, D, Iinter,
                                      layer0, layer1, n_experts)
        if h <= 0:
            raise HipError("mvllm_hip_slab_load failed: " + lib().mvllm_hip_last_error().decode())
        self.handle = h
        base, table = C.c_void_p(), C.c_void_p()
        stride, blob, nbl = np.zeros(1, np.int64), np.zeros(1, np.int64), np.zeros(1, np.int32)
        _check(lib().mvllm_hip_slab_info(h, C.byref(base), C.byref(table), _ptr(stride),
                                         _ptr(blob), _ptr(nbl)), "mvllm_hip_slab_info")
        self.base, self.table = base.value, table.value
        self.stride, self.blob_bytes, self.n_blobs = int(stride[0]), int(blob[0]), int(nbl[0])
        self.fmt, self.D, self.I = fmt, D, Iinter
        self.layer0, self.n_experts = layer0, n_experts

    def blob(self, layer, e):
        return self.base + ((layer - self.layer0) * self.n_experts + e) * self.stride

    def free(self):
        if self.handle:
            _check(lib().mvllm_hip_slab_free(self.handle), "mvllm_hip_slab_free")
            self.handle = 0


def prefetch(layers, eids, host_blobs, nbytes):
    """mvllm_hip_prefetch: -> copies enqueued."""
    n = len(eids)
    la, ea = np.asarray(layers, np.int32), np.asarray(eids, np.int32)
    by = np.asarray(nbytes, np.uint64)
    r = lib().mvllm_hip_prefetch(n, _ptr(la), _ptr(ea), _ptr_array(list(host_blobs)), _ptr(by))
    if r < 0:
        raise HipError("mvllm_hip_prefetch failed: " + lib().mvllm_hip_last_error().decode())
    return r


def repin(pairs):
    a = np.asarray(pairs, np.int32).reshape(-1, 2)
    r = lib().mvllm_hip_repin(len(a), _ptr(a))
    if r < 0:
        raise HipError("mvllm_hip_repin failed: " + lib().mvllm_hip_last_error().decode())
    return r


def tier_table(layer, n_experts, table_dev, stream=None):
    """-> number of resident entries written into table_dev (enqueued on stream)."""
    nres = np.zeros(1, np.int32)
    _check(lib().mvllm_hip_tier_table(layer, n_experts, _ptr(table_dev), _ptr(nres),
                                      _stream(stream)), "mvllm_hip_tier_table")
    return int(nres[0])


def tier_table_done(layer, stream=None):
    _check(lib().mvllm_hip_tier_table_done(layer, _stream(stream)), "mvllm_hip_tier_table_done")
