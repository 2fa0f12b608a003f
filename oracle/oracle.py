"""ctypes front end to the CPU parity checker (TEST INFRASTRUCTURE ONLY).

Loads ``oracle/liboracle.so`` (the C restatement in moe_oracle.c) and, when it
was built, ``oracle/_ref/libmvllm_ref.so`` (the reference's own sources compiled
with oracle/ref_shim.cpp).  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg import this module; the product path never does.

Both libraries expose the same functions (prefix ``orc_`` or ``ref_``), so
:class:`CpuMoe` wraps either one with numpy-friendly signatures.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmvllm_ref.so")

_f = C.c_float
_i = C.c_int
_p = C.c_void_p
_pp = C.POINTER(C.c_void_p)


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _ptr_array(arrs):
    """Host array of pointers (None entries become NULL); keeps arrs alive via closure."""
    arr = (C.c_void_p * len(arrs))()
    for i, a in enumerate(arrs):
        arr[i] = None if a is None else a.ctypes.data
    return arr


class CpuMoe:
    """numpy wrapper over liboracle.so (prefix 'orc') or _ref (prefix 'ref')."""

    def __init__(self, which: str = "oracle"):
        path, self.pfx = (ORACLE_SO, "orc") if which == "oracle" else (REF_SO, "ref")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = C.CDLL(path)
        self.which = which
        L, p = self.lib, self.pfx
        sig = {
            "moe_block": (_i, [_i, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _pp, _p, _p, _p, _p,
                               _p, _p, _i, _i, _f, _f]),
            "matmul_f32": (None, [_p, _p, _p, _i, _i, _i]),
            "matmul_int4_g64": (None, [_p, _p, _p, _p, _i, _i, _i]),
            "matmul_mxfp4": (None, [_p, _p, _p, _p, _i, _i, _i]),
            "matmul_int8_row": (None, [_p, _p, _p, _p, _i, _i, _i]),
            "sigmoid": (_f, [_f]),
            "clamped_swiglu": (_f, [_f, _f, _f]),
            "situ_glu": (_f, [_f, _f, _f, _f]),
            "mx4_lut": (_f, [_i]),
            "mx4_scale": (_f, [C.c_uint8]),
            "moe_topk": (_i, [_p, _i, _i, _p, _p, _p]),
            "moe_union_ids": (_i, [_p, _i, _i, _p, _i]),
            "moe_topk_batch": (_i, [_p, _i, _i, _i, _p, _p, _p]),
            "bf16_round": (_f, [_f]),
            "e8m0_decode": (_f, [C.c_uint8]),
            "e2m1_decode": (_f, [C.c_uint8]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, f"{p}_{name}")
            fn.restype, fn.argtypes = res, args
        if p == "orc":
            for name, (res, args) in {
                "apply_act": (None, [_p, _p, _i, _i, _f, _f]),
                "dequant_int4_g64": (None, [_p, _p, _p, _i, _i]),
                "dequant_mxfp4": (None, [_p, _p, _p, _i, _i]),
                "moe_segments": (_i, [_p, _p, _i, _i, _p, _p, _p, _p, _p, _i, _i, _p]),
                "fp4_activation_qdq": (_i, [_p, _p, _p, _i, _i, _p]),
                "rmsnorm": (None, [_p, _p, _p, _i, _f]),
                "route": (None, [_p, _p, _p, _i, _i, _i, _f, _p, _p]),
                "moe_block_fp4act": (_i, [_i, _i, _i, _i, _i, _pp, _pp, _pp, _pp, _pp, _pp, _p,
                                          _p, _p, _p, _p, _p, _i, _i, _f, _f]),
            }.items():
                fn = getattr(L, f"orc_{name}")
                fn.restype, fn.argtypes = res, args
        else:
            L.ref_fp4_activation_qdq.restype = _i
            L.ref_fp4_activation_qdq.argtypes = [_p, _p, _p, _i, _i]
            for name, args in {"quantize_int4_g64": [_p, _i, _i, _p, _p],
                               "quantize_int8_row": [_p, _i, _i, _p, _p],
                               "pack_mxfp4": [_p, _i, _i, _p, _p],
                               "silu_mul": [_p, _p, _i],
                               "bf16_round_array": [_p, _i],
                               "rmsnorm": [_p, _p, _p, _i, _f],
                               "norm_route": [_p, _p, _i, _f, _p, _p, _i, _i, _f, _p, _p,
                                              _p]}.items():
                fn = getattr(L, f"ref_{name}")
                fn.restype, fn.argtypes = None, args

    def fn(self, name):
        return getattr(self.lib, f"{self.pfx}_{name}")

    # ---- scalar / small helpers -------------------------------------------
    def sigmoid(self, x):
        return self.fn("sigmoid")(x)

    def clamped_swiglu(self, g, u, a):
        return self.fn("clamped_swiglu")(g, u, a)

    def situ_glu(self, g, u, b1, b2):
        return self.fn("situ_glu")(g, u, b1, b2)

    def bf16_round(self, v):
        return self.fn("bf16_round")(v)

    def rmsnorm(self, x, w, eps):
        """quant::rmsnorm of each row of x (w may be None)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        n = x.shape[-1]
        wp = None if w is None else np.ascontiguousarray(w, np.float32)
        for r in range(x.size // n):
            self.fn("rmsnorm")(x.ctypes.data + 4 * n * r, None if wp is None else wp.ctypes.data,
                               y.ctypes.data + 4 * n * r, n, eps)
        return y

    def route(self, x, w, bias, k, rscale=1.0):
        """cpu_route of each row of x (oracle only): -> idx [rows, k], wt [rows, k]."""
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        E, D = w.shape
        rows = x.size // D
        idx = np.zeros((rows, k), np.int32)
        wt = np.zeros((rows, k), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        for r in range(rows):
            self.fn("route")(x.ctypes.data + 4 * D * r, w.ctypes.data,
                             None if b is None else b.ctypes.data, D, E, k, rscale,
                             idx.ctypes.data + 4 * k * r, wt.ctypes.data + 4 * k * r)
        return idx, wt

    def norm_route(self, x, post_ln, eps, w, bias, k, rscale=1.0):
        """_ref only: metal_ops::layer_decode_full's host path on one row x:
        -> (nrm = rmsnorm(x, post_ln), idx, wt = cpu_route(nrm))."""
        x = np.array(x, np.float32, copy=True)
        w = np.ascontiguousarray(w, np.float32)
        E, D = w.shape
        nrm = np.zeros(D, np.float32)
        idx = np.zeros(k, np.int32)
        wt = np.zeros(k, np.float32)
        p = None if post_ln is None else np.ascontiguousarray(post_ln, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.ref_norm_route(x.ctypes.data, None if p is None else p.ctypes.data, D, eps,
                                w.ctypes.data, None if b is None else b.ctypes.data, E, k,
                                rscale, nrm.ctypes.data, idx.ctypes.data, wt.ctypes.data)
        return nrm, idx, wt

    def bf16_round_array(self, x):
        """The reference's bf16_round_array (src/quant/bf16.cpp:36-41) on a copy of x
        (f32 bit patterns pass through unchanged, NaN payloads included); _ref only."""
        a = np.array(x, dtype=np.float32, copy=True)
        self.lib.ref_bf16_round_array(a.ctypes.data, a.size)
        return a

    # ---- GEMMs ---------------------------------------------------------------
    def matmul(self, fmt, x, w, scales=None):
        """y[S,O] for fmt 0 (w f32 [O,I]), 4 (w packed u8 [O,(I+1)//2], scales f32), 7, or
        8 (QuantMat's int8 rows: w int8 [O,I], scales f32 [O])."""
        x = np.ascontiguousarray(x, np.float32)
        S, I = x.shape
        O = w.shape[0]
        y = np.zeros((S, O), np.float32)
        if fmt == 0:
            self.fn("matmul_f32")(_ptr(y), _ptr(x), _ptr(np.ascontiguousarray(w, np.float32)),
                                  S, I, O)
        elif fmt == 4:
            self.fn("matmul_int4_g64")(_ptr(y), _ptr(x), _ptr(w), _ptr(scales), S, I, O)
        elif fmt == 8:
            self.fn("matmul_int8_row")(_ptr(y), _ptr(x), _ptr(np.ascontiguousarray(w, np.int8)),
                                       _ptr(np.ascontiguousarray(scales, np.float32)), S, I, O)
        else:
            self.fn("matmul_mxfp4")(_ptr(y), _ptr(x), _ptr(w), _ptr(scales), S, I, O)
        return y

    # ---- moe_block -----------------------------------------------------------
    def moe_block(self, nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S,
                  act=0, act_a=0.0, act_b=0.0, qgs=0):
        """Calls <pfx>_moe_block; lists g/u/d/gs/us/ds hold per-expert arrays or None.

        Any of the list arguments may itself be None (a NULL pointer array).
        ``out`` is accumulated in place.  Returns the int result (1 ran, 0 fall back).
        """
        pa = [None if L is None else _ptr_array(L) for L in (g, u, d, gs, us, ds)]
        return self.fn("moe_block")(
            nb, D, Iinter, fmt, qgs, *pa, _ptr(xg), _ptr(xoff), _ptr(nr), _ptr(rows), _ptr(rw),
            _ptr(out), S, act, act_a, act_b)

    def moe_block_fp4act(self, nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw,
                         out, S, act=0, act_a=0.0, act_b=0.0, qgs=0):
        """moe_block with MXFP4-quantized GEMM inputs (the native-FP4 path's checker;
        restatement only)."""
        pa = [None if L is None else _ptr_array(L) for L in (g, u, d, gs, us, ds)]
        return self.lib.orc_moe_block_fp4act(
            nb, D, Iinter, fmt, qgs, *pa, _ptr(xg), _ptr(xoff), _ptr(nr), _ptr(rows), _ptr(rw),
            _ptr(out), S, act, act_a, act_b)

    def moe_topk(self, choice, k, mix=None):
        choice = np.ascontiguousarray(choice, np.float32)
        n = choice.shape[0]
        idx = np.full(max(k, 1), -7, np.int32)
        w = np.zeros(max(k, 1), np.float32)
        kk = self.fn("moe_topk")(_ptr(choice), n, k, _ptr(idx), _ptr(w),
                                 _ptr(None if mix is None else np.ascontiguousarray(mix, np.float32)))
        return kk, idx[:max(kk, 0)], w[:max(kk, 0)]

    def moe_topk_batch(self, choice, k, mix=None):
        """moe_topk over every row of choice [T, n] in one native call."""
        choice = np.ascontiguousarray(choice, np.float32)
        T, n = choice.shape
        idx = np.full((T, max(k, 1)), -7, np.int32)
        w = np.zeros((T, max(k, 1)), np.float32)
        kk = self.fn("moe_topk_batch")(_ptr(choice), T, n, k, _ptr(idx), _ptr(w),
                                       _ptr(None if mix is None else np.ascontiguousarray(mix, np.float32)))
        return kk, idx[:, :max(kk, 0)], w[:, :max(kk, 0)]

    def moe_union_ids(self, idx, n_tok, topk, cap):
        idx = np.ascontiguousarray(idx, np.int32)
        out = np.full(max(cap, 1), -7, np.int32)
        n = self.fn("moe_union_ids")(_ptr(idx), n_tok, topk, _ptr(out), cap)
        return out[:n]

    def e8m0_decode(self, v):
        return self.fn("e8m0_decode")(v)

    def e2m1_decode(self, v):
        return self.fn("e2m1_decode")(v)

    def fp4_activation_qdq(self, x, block):
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[0]
        out = np.zeros(n, np.float32)
        sc = np.zeros((n + block - 1) // block, np.uint8)
        if self.pfx == "orc":
            codes = np.zeros(n, np.uint8)
            rc = self.lib.orc_fp4_activation_qdq(_ptr(out), _ptr(sc), _ptr(x), n, block,
                                                 _ptr(codes))
            return rc, out, sc, codes
        rc = self.lib.ref_fp4_activation_qdq(_ptr(out), _ptr(sc), _ptr(x), n, block)
        return rc, out, sc, None

    # ---- oracle-only -----------------------------------------------------------
    def dequant(self, fmt, packed, scales, O, I):
        w = np.zeros((O, I), np.float32)
        f = self.lib.orc_dequant_int4_g64 if fmt == 4 else self.lib.orc_dequant_mxfp4
        f(_ptr(w), _ptr(packed), _ptr(scales), O, I)
        return w

    def moe_segments(self, idx, wt, n_tok, topk, cap_experts):
        idx = np.ascontiguousarray(idx, np.int32)
        wt = np.ascontiguousarray(wt, np.float32)
        cap_rows = max(n_tok * topk, 1)
        eids = np.zeros(cap_experts, np.int32)
        xoff = np.zeros(cap_experts, np.int32)
        nr = np.zeros(cap_experts, np.int32)
        rows = np.zeros(cap_rows, np.int32)
        rw = np.zeros(cap_rows, np.float32)
        nrows = C.c_int(0)
        nb = self.lib.orc_moe_segments(_ptr(idx), _ptr(wt), n_tok, topk, _ptr(eids), _ptr(xoff),
                                       _ptr(nr), _ptr(rows), _ptr(rw), cap_experts, cap_rows,
                                       C.cast(C.pointer(nrows), C.c_void_p))
        j = nrows.value
        return nb, eids[:nb], xoff[:nb], nr[:nb], rows[:j], rw[:j]

    def apply_act(self, g, u, act, a, b):
        g = np.ascontiguousarray(g, np.float32).copy()
        u = np.ascontiguousarray(u, np.float32)
        self.lib.orc_apply_act(_ptr(g), _ptr(u), g.size, act, a, b)
        return g


def have_ref() -> bool:
    return os.path.exists(REF_SO)
