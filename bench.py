"""moe_block benchmark on one MI355X.

Headline workload: config c4, the largest single-GPU configuration (K3-style MXFP4
prefill, D=7168, I=2048, 384 experts, top-8, T=2048 tokens, Zipf(1.1) routing, SiTU)
through mvllm_hip_moe_block_dev with weights, activations and output resident in HBM.
One step = one call: the bf16 grouped GEMM over the token-sorted expert segments (gate/up
+ activation, down) and the top-k combine in the reference's order.  The same run also
reports, under "extra": c4 on native MXFP4 activations (scaled FP4 matrix cores), c0,
c1 at T=1/4/16, c2 (resident, and through the drop-in host entry with 25% of its experts
staged from pinned host memory) and c3.  Every timed call reads its experts from a weight
pool of >= 4 GiB (a whole c3/c4 call reads >= 5.4 GB), so the 256 MB Infinity Cache
cannot serve repeated weights.

Prints ONE JSON line on stdout; details go to stderr.
  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--tokens T]
                  [--fp4act] [--no-extra] [--no-cpu]
"""
import argparse
import contextlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "micro-vllm_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E
FP4_PEAK_TFS = 10100.0    # dense MXFP4 matrix cores
BF16_PEAK_TFS = 2500.0    # dense bf16 matrix cores
METRIC = "moe_block tokens/s + effective weight GB/s (decode), MFMA util (prefill)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_bytes(workload, kernel):
    """HBM bytes per call of `kernel` in `workload` from rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs (profiles/traffic.json, each counter calibrated by a copy of known size), or None
    when that pair has not been measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    v = d.get(workload, {}).get(kernel)
    return None if v is None else v.get("bytes")


def expert_bytes(fmt, D, I):
    """Algorithmic bytes of one expert in the reference layout: (gate + up, down)."""
    gq, sb = (64, 4) if fmt == 4 else (32, 1)
    gu = 2 * (I * ((D + 1) // 2) + I * ((D + gq - 1) // gq) * sb)
    dn = D * ((I + 1) // 2) + D * ((I + gq - 1) // gq) * sb
    return gu, dn


def binding_roof_us(nr, bytes_e, flops_per_row, peak_tfs):
    """t_lb = sum over experts of max(bytes_e / HBM peak, flops_e / matrix-core peak), us."""
    t = 0.0
    for n in nr:
        t += max(bytes_e / (HBM_PEAK_GBS * 1e9), flops_per_row * float(n) / (peak_tfs * 1e12))
    return t * 1e6


def build_pool(torch, mvllm_hip, fmt, D, I, n_blobs, seed):
    """n_blobs expert blobs in the reference layout, generated on the GPU."""
    from mvllm_hip import synth
    nbytes, off = mvllm_hip.expert_geom(fmt, D, I)
    pool, stride = synth.device_pool(torch, fmt, D, I, n_blobs, seed, (nbytes, off))
    return pool, stride, off, nbytes


class Pool:
    """A weight pool for one configuration: `layers` layers of the workload's nb experts,
    rotated per step, together at least pool_gb (or one layer when that is larger)."""

    def __init__(self, np, torch, mvllm_hip, w, fmt, D, I, pool_gb, seed=1234):
        nbytes, _ = mvllm_hip.expert_geom(fmt, D, I)
        self.layers = max(1, int(np.ceil(pool_gb * 2**30 / (nbytes * w.nb))))
        self.n_blobs = self.layers * w.nb
        self.pool, self.stride, self.off, self.nbytes = build_pool(torch, mvllm_hip, fmt, D, I,
                                                                   self.n_blobs, seed)
        base = self.pool.data_ptr()
        order = (0, 2, 4, 1, 3, 5)  # geometry offsets: gate_p gate_s up_p up_s down_p down_s
        self.lists = []
        for layer in range(self.layers):
            ptrs = [[], [], [], [], [], []]
            for i in range(w.nb):
                b = base + (layer * w.nb + i) * self.stride
                for slot, oi in enumerate(order):
                    ptrs[slot].append(b + int(self.off[oi]))
            self.lists.append(mvllm_hip.prepare_lists(*ptrs))
        self.gib = self.n_blobs * self.nbytes / 2**30


def measure(np, torch, mvllm_hip, synth, name, T, steps, warmup, pool_gb, fp4act=False,
            pool=None, w=None, cpu_seconds=0.0):
    """Times `steps` moe_block_dev calls of workload (name, T) after `warmup`, then a second
    pass with the library's per-phase HIP events (recorded on the stream the kernels run
    on).  Returns (record, pool, workload)."""
    cfg = synth.CONFIGS[name]
    D, I, fmt = cfg["D"], cfg["I"], cfg["fmt"]
    if w is None:
        w = synth.make_workload(name, T=T, with_experts=False)
    if pool is None:
        pool = Pool(np, torch, mvllm_hip, w, fmt, D, I, pool_gb)
    mvllm_hip.set_option("fp4act", 1 if fp4act else 0)
    xg = torch.from_numpy(w.xg).cuda()
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    addr = [xg.data_ptr()] + [a.ctypes.data for a in (w.xoff, w.nr, w.rows, w.rw)] + \
        [out.data_ptr()]

    def step(s):
        mvllm_hip.moe_block_dev(w.nb, D, I, fmt, None, None, None, None, None, None, *addr[:5],
                                addr[5], T, w.act, w.a, w.b,
                                prepared=pool.lists[s % pool.layers])

    for s in range(warmup):
        step(s)
    torch.cuda.synchronize()
    # timed region: `steps` calls bracketed by synchronize; torch's stream is the null
    # stream, which the library's kernels run on
    st0 = mvllm_hip.stats()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for s in range(steps):
        step(s)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / steps
    st1 = mvllm_hip.stats()
    host_us = (st1["host_ms"] - st0["host_ms"]) / steps * 1e3
    wait_us = (st1["host_wait_ms"] - st0["host_wait_ms"]) / steps * 1e3
    # the host's own work per call (plan + launches) with the device idle: in the loop
    # above the host runs ahead and also waits on a full launch queue.  The median of 20
    # calls, each after a synchronize: the first calls after the timed loop pay a thread
    # wake-up several times the steady cost
    n_iso = min(steps, 20)
    iso, plan = [], []
    for s in range(n_iso):
        torch.cuda.synchronize()
        h0 = mvllm_hip.stats()
        step(s)
        h1 = mvllm_hip.stats()
        iso.append(h1["host_ms"] - h0["host_ms"])
        plan.append(h1["host_plan_ms"] - h0["host_plan_ms"])
    torch.cuda.synchronize()
    iso_us = float(np.median(iso)) * 1e3
    plan_us = float(np.median(plan)) * 1e3
    # per-phase kernel durations: a second pass with HIP events around each phase
    mvllm_hip.set_option("timing", 1)
    mvllm_hip.stats_reset()
    for s in range(steps):
        step(s)
    torch.cuda.synchronize()
    st = mvllm_hip.stats()
    mvllm_hip.set_option("timing", 0)
    mvllm_hip.set_option("fp4act", 0)
    ph = {k: st["ms_" + k] / steps * 1e3 for k in ("prep", "gate_up", "down", "combine")}

    nr = [int(n) for n in w.nr]
    rows = int(sum(nr))
    gemm = max(nr) > 16 or fp4act
    if fp4act and fmt == 7:
        dtype, peak = "mxfp4", FP4_PEAK_TFS
    else:
        dtype, peak = ("bf16" if gemm else "bf16x2"), BF16_PEAK_TFS
    b_gu, b_dn = expert_bytes(fmt, D, I)
    wbytes = w.nb * (b_gu + b_dn)
    flops = 6.0 * D * I * rows
    t_gu = ph["gate_up"]
    gu_gbs = w.nb * b_gu / (t_gu * 1e-6) / 1e9
    lb_gu = binding_roof_us(nr, b_gu, 4.0 * D * I, peak)
    lb_call = binding_roof_us(nr, b_gu + b_dn, 6.0 * D * I, peak)
    wl = f"{name} T={T}" + (" fp4act" if fp4act else "")
    kern = ("k_gemm_fp4 + k_gemm gate/up" if fp4act else
            "k_gemm + k_gemm_wide gate/up" if fmt == 7 else "k_gemm gate/up") if gemm else \
        "k_mfma_dec gate/up"
    rec = {
        "workload": f"{name} {cfg['desc']}, T={T}" + (", native MXFP4 activations" if fp4act else ""),
        "value": round(T / (ms_step * 1e-3), 2), "unit": "tokens/s",
        "ms_per_step": round(ms_step, 6), "wall_ms_per_step": round(wall / steps * 1e3, 6),
        "host_us_per_call": round(iso_us, 1), "host_plan_us_per_call": round(plan_us, 1),
        "host_loop_us_per_call": round(host_us - wait_us, 1),
        "host_wait_us_per_call": round(wait_us, 1), "dtype": dtype,
        "experts": int(w.nb), "rows": rows, "max_rows_per_expert": int(max(nr)),
        "weight_gbps": round(wbytes / (ms_step * 1e-3) / 1e9, 1),
        "weight_bytes": int(wbytes), "flops": flops,
        "mfma_util": {"bf16": round(flops / (ms_step * 1e-3) / (BF16_PEAK_TFS * 1e12), 5),
                      "fp4": round(flops / (ms_step * 1e-3) / (FP4_PEAK_TFS * 1e12), 5)},
        "phases_us": {k: round(v, 3) for k, v in ph.items()},
        "kernel_sum_us": round(sum(ph.values()), 3),
        "roofline": {
            "bound": "hbm", "kernel": kern + (" (all row classes of one call)" if gemm else ""),
            "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes(wl, "gate_up"),
            "bytes_per_launch": int(w.nb * b_gu), "avg_launch_us": round(t_gu, 3),
            "binding": {"t_lb_us": round(lb_gu, 2), "frac": round(lb_gu / t_gu, 4),
                        "peak_tflops": peak,
                        "rule": "sum over experts of max(gate/up bytes / 8 TB/s, "
                                "4 D I rows / matrix-core peak)"},
        },
        "call_binding": {"t_lb_us": round(lb_call, 2), "t_us": round(ms_step * 1e3, 2),
                         "frac": round(lb_call / (ms_step * 1e3), 4)},
        "pool_gib": round(pool.gib, 2),
    }
    log(f"[{wl}] step {ms_step*1e3:.1f} us (wall {wall/steps*1e6:.1f} us, host {iso_us:.1f} "
        f"us/call with the device idle (median), {plan_us:.1f} of it before the launches; in the loop {host_us - wait_us:.1f} us/call + "
        f"{wait_us:.1f} us blocked on plan slots): prep {ph['prep']:.1f}, gate/up {t_gu:.1f}, down "
        f"{ph['down']:.1f}, combine {ph['combine']:.1f} us; gate/up {gu_gbs:.0f} GB/s "
        f"(binding roof {lb_gu:.1f} us, {lb_gu/t_gu:.3f}); call {lb_call/(ms_step*1e3):.3f} "
        f"of its binding roof; MFMA util bf16 {rec['mfma_util']['bf16']:.3f} fp4 "
        f"{rec['mfma_util']['fp4']:.4f}")
    if cpu_seconds > 0:
        rec["cpu_baseline"] = cpu_baseline(np, torch, w, pool.pool, pool.stride, pool.off, fmt,
                                           D, I, T, cpu_seconds)
    del xg, out
    return rec, pool, w


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4")
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--mode", type=int, default=0)
    ap.add_argument("--opt", action="append", default=[], metavar="KEY=VALUE",
                    help="extra mvllm_hip_set_option settings (e.g. dec_ks=2)")
    ap.add_argument("--fp4act", action="store_true",
                    help="headline on native MXFP4 activations (scaled-FP4 matrix cores)")
    ap.add_argument("--pool-gb", type=float, default=4.5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="only the headline workload (profiling runs: no other workloads, "
                         "no c4 hot-segment calls)")
    ap.add_argument("--probe-sizes", action="store_true",
                    help="also time the stream-read probe at launch-sized reads (8 MiB .. "
                         "1 GiB, each repetition at a new offset of the pool)")
    ap.add_argument("--pipeline", action="store_true",
                    help="only the c2 layer pipeline (HBM tier fed like the store feeds it)")
    ap.add_argument("--staged", type=float, default=None, metavar="MISS_RATE",
                    help="only the drop-in host entry with the HBM expert tier: this fraction "
                         "of each step's experts is copied from pinned host memory by the call")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the expert-parallel sharding is a design note); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import mvllm_hip
    from mvllm_hip import synth

    cfg = dict(synth.CONFIGS[args.config])
    T = args.tokens or cfg["T"]
    mvllm_hip.init(0)
    mvllm_hip.set_option("mode", args.mode)
    for kv in args.opt:
        k, v = kv.split("=", 1)
        if not mvllm_hip.set_option(k, int(v)):
            raise SystemExit(f"option {kv} refused")
    if args.pipeline:
        print(json.dumps(layer_pipeline(np, torch, mvllm_hip, synth,
                                        dict(synth.CONFIGS["c2"]))), flush=True)
        return
    if args.staged is not None:
        print(json.dumps(staged(args, np, torch, mvllm_hip, synth, cfg, T, args.steps,
                                args.warmup, args.staged,
                                0.0 if args.no_cpu else args.cpu_seconds)), flush=True)
        return

    cpu_s = 0.0 if args.no_cpu else args.cpu_seconds
    head, pool, w = measure(np, torch, mvllm_hip, synth, args.config, T, args.steps,
                            args.warmup, args.pool_gb, fp4act=args.fp4act, cpu_seconds=cpu_s)

    # achievable HBM streaming-read rate on this box: coalesced 16-byte loads over the
    # headline's weight pool (beyond the Infinity Cache), after one warm-up pass; and a
    # 1 GiB copy, whose known byte counts calibrate the FETCH_SIZE / WRITE_SIZE counters
    sink = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    probe_bytes = min((pool.pool.numel() // 4096) * 4096, 8 << 30)
    hbm_gbs = probe_bytes / mvllm_hip.membench(0, pool.pool, sink, probe_bytes, 0, 5) / 1e6
    copy_bytes = min(1 << 30, probe_bytes)
    dst = torch.empty(copy_bytes, dtype=torch.uint8, device="cuda")
    copy_gbs = 2 * copy_bytes / mvllm_hip.membench(1, pool.pool, dst, copy_bytes, 0, 3) / 1e6
    del dst
    log(f"HBM stream-read probe: {hbm_gbs:.0f} GB/s over {probe_bytes / 2**30:.2f} GiB; "
        f"copy probe {copy_gbs:.0f} GB/s (read + write) over {copy_bytes / 2**30:.2f} GiB")
    sizes = probe_sizes(np, mvllm_hip, pool.pool, sink, probe_bytes) if args.probe_sizes else {}

    extra = {}
    if args.config == "c4" and not args.no_extra:  # (profiling runs: the call alone)
        hot = hot_segments(np, torch, mvllm_hip, w, pool, cfg, T, args.steps, 2)
        if hot:
            extra["c4 hot segments"] = hot
        extra["c4 routed_dev"] = routed_prefill(np, torch, mvllm_hip, w, pool, cfg, T,
                                                args.steps, 2)
    if not args.no_extra:
        if args.config == "c4" and not args.fp4act:
            rec, _, _ = measure(np, torch, mvllm_hip, synth, "c4", T, args.steps, 2,
                                args.pool_gb, fp4act=True, pool=pool, w=w)
            extra["c4 T=%d fp4act" % T] = rec
        del pool
        torch.cuda.empty_cache()
        for name, t, steps in (("c3", 512, args.steps), ("c2", 1, 200), ("c1", 16, 200),
                               ("c1", 4, 200), ("c1", 1, 200), ("c0", 1, 200)):
            if (name, t) == (args.config, T):
                continue
            rec, p, _ = measure(np, torch, mvllm_hip, synth, name, t, steps, 20, args.pool_gb,
                                cpu_seconds=0.0 if args.no_cpu else 3.0)
            extra[f"{name} T={t}"] = rec
            del p
            torch.cuda.empty_cache()
        extra["c2 T=1 staged"] = staged(args, np, torch, mvllm_hip, synth,
                                        dict(synth.CONFIGS["c2"]), 1, 50, 5, 0.25, 0.0)
        extra["c2 layer pipeline"] = layer_pipeline(np, torch, mvllm_hip, synth,
                                                    dict(synth.CONFIGS["c2"]))
        route, scores = route_timing(torch, mvllm_hip, 2048, 384, 8)
        if not args.no_cpu:
            route["cpu_us_per_call"], route["cpu_kind"] = cpu_route_baseline(np, scores, 8)
        extra["route c4 shape"] = route
    else:
        del pool

    rec = {
        "metric": METRIC, "value": head["value"], "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded; weights random in the reference layouts, in a "
                f"{head['pool_gib']:.1f} GiB pool; activations N(0,1) rounded to bf16)",
        "config": {"workload": head["workload"], "D": cfg["D"], "I": cfg["I"], "E": cfg["E"],
                   "topk": cfg["k"], "T": T, "fmt": cfg["fmt"], "routing": cfg["routing"],
                   "experts_per_step": head["experts"], "rows": head["rows"],
                   "mode": args.mode, "fp4act": bool(args.fp4act), "options": args.opt},
        "weight_gbps": head["weight_gbps"], "mfma_util": head["mfma_util"],
        "roofline": head["roofline"], "call_binding": head["call_binding"],
        "phases_us": head["phases_us"], "kernel_sum_us": head["kernel_sum_us"],
        "host_us_per_call": head["host_us_per_call"],
        "hbm_probe_gbps": round(hbm_gbs, 1), "hbm_copy_probe_gbps": round(copy_gbs, 1),
        **({"hbm_probe_by_size_mib": sizes} if sizes else {}),
        "cpu_baseline": head.get("cpu_baseline"),
        "extra": extra,
    }
    print(json.dumps(rec), flush=True)


def routed_prefill(np, torch, mvllm_hip, w, pool, cfg, T, steps, warmup):
    """The device-resident block at the c4 shape: mvllm_hip_moe_block_routed_dev on the
    workload's segments in device memory (as mvllm_hip_moe_route_dev leaves them) with a
    device table of the pool layer's blobs, against the host-planned moe_block_dev call on
    the same segments and the same rotation of pool layers (HIP events around `steps`
    calls of each, after `warmup`), in the default bf16 arithmetic and with native MXFP4
    activations (option fp4act).  Both write the same out rows; the routed call plans on
    the device and launches its grids for the caps (cap_experts = E, cap_rows = T k)."""
    D, I, fmt, E = cfg["D"], cfg["I"], cfg["fmt"], cfg["E"]
    i32 = dict(dtype=torch.int32, device="cuda")
    n_rows = int(np.sum(w.nr))
    counts = torch.tensor([w.nb, n_rows], **i32)
    eids = torch.from_numpy(np.ascontiguousarray(w.eids, np.int32)).cuda()
    xoff = torch.from_numpy(np.ascontiguousarray(w.xoff, np.int32)).cuda()
    nr = torch.from_numpy(np.ascontiguousarray(w.nr, np.int32)).cuda()
    rows = torch.from_numpy(np.ascontiguousarray(w.rows, np.int32)).cuda()
    rw = torch.from_numpy(np.ascontiguousarray(w.rw, np.float32)).cuda()
    x = torch.from_numpy(np.ascontiguousarray(w.x, np.float32)).cuda()
    xg = torch.from_numpy(w.xg).cuda()
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    b0 = pool.pool.data_ptr()
    tables = []
    for layer in range(pool.layers):
        t = np.zeros(E, np.int64)
        for i in range(w.nb):
            t[int(w.eids[i])] = b0 + (layer * w.nb + i) * pool.stride
        tables.append(torch.from_numpy(t).cuda())
    status = torch.zeros(1, **i32)

    def routed(s):
        mvllm_hip.moe_block_routed_dev(D, I, fmt, tables[s % len(tables)], E, counts, eids, xoff,
                                       nr, rows, rw, x, out, T, w.act, w.a, w.b, status=status)

    def planned(s):
        mvllm_hip.moe_block_dev(w.nb, D, I, fmt, None, None, None, None, None, None, xg,
                                w.xoff, w.nr, w.rows, w.rw, out, T, w.act, w.a, w.b,
                                prepared=pool.lists[s % pool.layers])

    rec = {}
    for sfx, fp4 in (("", 0), ("_fp4act", 1)):
        if not mvllm_hip.set_option("fp4act", fp4):
            raise SystemExit("set_option fp4act failed")
        try:
            for key, fn in (("routed_dev_us", routed), ("host_planned_us", planned)):
                for s in range(warmup):
                    fn(s)
                torch.cuda.synchronize()
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                for s in range(steps):
                    fn(s)
                e1.record()
                torch.cuda.synchronize()
                rec[key + sfx] = round(e0.elapsed_time(e1) / steps * 1e3, 2)
        finally:
            mvllm_hip.set_option("fp4act", 0)
        if int(status.cpu()[0]) != 0:
            raise SystemExit("routed_dev reported status %d" % int(status.cpu()[0]))
        rec["ratio" + sfx] = round(rec["routed_dev_us" + sfx] / rec["host_planned_us" + sfx], 4)
        log(f"c4 device-resident block{sfx}: {rec['routed_dev_us' + sfx]:.1f} us per call, "
            f"host-planned {rec['host_planned_us' + sfx]:.1f} us ({rec['ratio' + sfx]:.3f})")
    return rec


def hot_segments(np, torch, mvllm_hip, w, pool, cfg, T, steps, warmup, min_rows=332):
    """Matrix-core utilisation of the compute-bound segments: the experts of the workload
    with >= min_rows rows (at c4, the experts that are compute-bound even on the FP4 peak),
    as one moe_block_dev call over those experts only (their rows, combine weights and out
    rows as in the full call), timed with events in the default bf16 arithmetic and with
    native MXFP4 activations.  FLOPs = 6 D I rows; utilisation against the dense bf16 and
    FP4 peaks."""
    D, I, fmt = cfg["D"], cfg["I"], cfg["fmt"]
    sel = [i for i in range(w.nb) if int(w.nr[i]) >= min_rows]
    if not sel:
        return None
    nr = np.ascontiguousarray(w.nr[sel], np.int32)
    xoff = np.ascontiguousarray(w.xoff[sel], np.int32)
    base = np.concatenate(([0], np.cumsum(w.nr)))
    pick = np.concatenate([np.arange(base[i], base[i + 1]) for i in sel])
    rows = np.ascontiguousarray(w.rows[pick], np.int32)
    rw = np.ascontiguousarray(w.rw[pick], np.float32)
    lists = []
    order = (0, 2, 4, 1, 3, 5)
    b0 = pool.pool.data_ptr()
    for layer in range(pool.layers):
        ptrs = [[b0 + (layer * w.nb + i) * pool.stride + int(pool.off[o]) for i in sel]
                for o in order]
        lists.append(mvllm_hip.prepare_lists(*ptrs))
    xg = torch.from_numpy(w.xg).cuda()
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    flops = 6.0 * D * I * float(nr.sum())
    rec = {"min_rows": min_rows, "experts": len(sel), "rows": int(nr.sum()),
           "rows_per_expert": [int(n) for n in nr], "flops": flops}
    for fp4 in (False, True):
        mvllm_hip.set_option("fp4act", 1 if fp4 else 0)

        def step(s):
            mvllm_hip.moe_block_dev(len(sel), D, I, fmt, None, None, None, None, None, None, xg,
                                    xoff, nr, rows, rw, out, T, w.act, w.a, w.b,
                                    prepared=lists[s % len(lists)])
        for s in range(warmup):
            step(s)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for s in range(steps):
            step(s)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        tf = flops / (ms * 1e-3) / 1e12
        key = "fp4act" if fp4 else "bf16"
        rec[key] = {"us_per_call": round(ms * 1e3, 2), "tflops": round(tf, 1),
                    "mfma_util_bf16": round(tf / BF16_PEAK_TFS, 4),
                    "mfma_util_fp4": round(tf / FP4_PEAK_TFS, 4)}
        log(f"hot segments (>= {min_rows} rows: {len(sel)} experts, {int(nr.sum())} rows), "
            f"{key}: {ms*1e3:.1f} us per call, {tf:.0f} TFLOP/s = "
            f"{tf / BF16_PEAK_TFS:.3f} of the bf16 peak, {tf / FP4_PEAK_TFS:.3f} of the FP4 peak")
    mvllm_hip.set_option("fp4act", 0)
    del xg, out
    return rec


def probe_sizes(np, mvllm_hip, pool, sink, probe_bytes):
    """Stream-read probe at launch-sized reads; each size read 20 times at new offsets of
    the pool (no Infinity Cache hits), median of the last 16."""
    sizes, flat = {}, pool.view(-1)
    for mib in (8, 16, 32, 64, 128, 192, 256, 512, 1024):
        nb = mib << 20
        if nb * 4 > probe_bytes:
            break
        ts, offset = [], 0
        for r in range(20):
            if offset + nb > probe_bytes:
                offset = 0
            ms = mvllm_hip.membench(0, flat[offset:offset + nb], sink, nb, 0, 1)
            offset += nb
            if r >= 4:
                ts.append(ms)
        t = float(np.median(ts))
        sizes[mib] = {"us": round(t * 1e3, 2), "gbps": round(nb / t / 1e6, 1)}
        log(f"  read {mib:5d} MiB in one launch: {t*1e3:8.2f} us, {nb / t / 1e6:7.0f} GB/s")
    return sizes


def route_timing(torch, mvllm_hip, T, E, k, reps=100):
    """GPU time per call of mvllm_hip_moe_route_dev (moe_topk of every token, then the
    segments) on N(0,1) router scores (weights from their sigmoid), HIP events on the
    null stream the calls are enqueued on.  Returns the record and the scores (for the
    host baseline)."""
    g = torch.Generator(device="cuda").manual_seed(7)
    choice = torch.randn((T, E), device="cuda", generator=g)
    mix = torch.sigmoid(choice)
    i32 = dict(dtype=torch.int32, device="cuda")
    idx, wt = torch.empty((T, k), **i32), torch.empty((T, k), dtype=torch.float32, device="cuda")
    work, counts = torch.empty(2 * E + 1, **i32), torch.empty(2, **i32)
    eids, xoff, nr = (torch.empty(E, **i32) for _ in range(3))
    rows, rw = torch.empty(T * k, **i32), torch.empty(T * k, dtype=torch.float32, device="cuda")
    a = [x.data_ptr() for x in (choice, mix, idx, wt, work, eids, xoff, nr, rows, rw, counts)]
    L = mvllm_hip.lib()

    def one():
        return L.mvllm_hip_moe_route_dev(a[0], a[1], T, E, k, a[2], a[3], a[4], a[5], a[6], a[7],
                                         a[8], a[9], E, T * k, a[10], None)
    for _ in range(10):
        if not one():
            raise SystemExit("device routing failed: " + L.mvllm_hip_last_error().decode())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        one()
    e1.record()
    torch.cuda.synchronize()
    nb, n_rows = (int(v) for v in counts.cpu())
    rec = {"us_per_call": round(e0.elapsed_time(e1) / reps * 1e3, 3), "n_tok": T, "n_exp": E,
           "k": k, "experts": nb, "rows": n_rows, "launches_per_call": 5}
    log(f"device routing (T={T}, E={E}, k={k}): {rec['us_per_call']:.2f} us per call")
    return rec, (choice.cpu().numpy(), mix.cpu().numpy())


def cpu_route_baseline(np, scores, k, budget_s=2.0):
    """The host routing on the same scores, one thread: moe_topk for every token in one
    native call (oracle/_ref build when present, else the C restatement), then the
    segments (C restatement), so the figure carries two ctypes calls, not one per token."""
    import oracle
    kind = "reference" if oracle.have_ref() else "port"
    topk = oracle.CpuMoe("ref" if kind == "reference" else "oracle")
    seg = oracle.CpuMoe("oracle")
    choice, mix = scores
    T, E = choice.shape
    with one_core():
        calls, t0 = 0, time.perf_counter()
        while True:
            _, idx, wt = topk.moe_topk_batch(choice, k, mix)
            seg.moe_segments(idx, wt, T, k, E)
            calls += 1
            if time.perf_counter() - t0 > budget_s:
                break
        t_call = (time.perf_counter() - t0) / calls
    return round(t_call * 1e6, 1), \
        f"{kind}; moe_topk over all tokens in one native call, then the segments"


def staged(args, np, torch, mvllm_hip, synth, cfg, T, steps, warmup, miss_rate, cpu_seconds):
    """One step = one drop-in mvllm_hip_moe_block call on host pointers (activations and
    output in host memory, as the engine calls it).  Expert blobs live in one pinned host
    buffer (the ExpertStore slots); most are promoted into the library's HBM tier at set-up,
    the rest are host-only, and each step draws round(miss_rate * nb) of its experts from
    them, so the call copies those blobs in on its copy stream while the resident experts
    compute.  Resident and host-only sets rotate over more than the Infinity Cache holds."""
    import ctypes
    D, I, fmt = cfg["D"], cfg["I"], cfg["fmt"]
    name = [k for k, v in synth.CONFIGS.items() if v["desc"] == cfg["desc"]][0]
    w = synth.make_workload(name, T=T, with_experts=False)
    nbytes, off = mvllm_hip.expert_geom(fmt, D, I)
    stride = (nbytes + 4095) // 4096 * 4096
    n_miss = int(round(miss_rate * w.nb))
    n_res = w.nb - n_miss
    r_res = max(n_res, int(np.ceil(1.2 * 2**30 / nbytes)))   # resident blobs (> 1 GiB)
    r_host = max(n_miss, 2 * n_miss * 4)                      # host-only blobs
    total = r_res + r_host
    L = mvllm_hip.lib()
    host = L.mvllm_hip_host_alloc(total * stride)
    if not host:
        raise SystemExit("pinned host allocation failed")
    pool, pstride, poff, _ = build_pool(torch, mvllm_hip, fmt, D, I, total, 1234)
    for b in range(total):  # reference layout, one slot per blob
        src = pool[b, :nbytes].cpu().numpy()
        ctypes.memmove(host + b * stride, src.ctypes.data, nbytes)
    for b in range(r_res):
        mvllm_hip.promote(host + b * stride, nbytes, 0, b)
    torch.cuda.synchronize()
    log(f"staged {name} T={T}: {w.nb} experts/step ({n_res} resident, {n_miss} misses), "
        f"{r_res} resident + {r_host} host-only blobs of {nbytes / 2**20:.2f} MiB")
    order = (0, 2, 4, 1, 3, 5)

    def lists(s):
        blobs = [(s * n_res + j) % r_res for j in range(n_res)] + \
                [r_res + (s * n_miss + j) % r_host for j in range(n_miss)]
        ptrs = [[], [], [], [], [], []]
        for b in blobs:
            for slot, oi in enumerate(order):
                ptrs[slot].append(host + b * stride + int(off[oi]))
        return ptrs

    out = np.zeros((T, D), np.float32)

    def step(s):
        out[:] = 0.0
        mvllm_hip.moe_block(w.nb, D, I, fmt, *lists(s), w.xg, w.xoff, w.nr, w.rows, w.rw, out,
                            T, w.act, w.a, w.b)

    for s in range(warmup):
        step(s)
    mvllm_hip.set_option("timing", 1)
    mvllm_hip.stats_reset()
    t0 = time.perf_counter()
    for s in range(steps):
        step(warmup + s)
    wall = (time.perf_counter() - t0) / steps
    st = mvllm_hip.stats()
    mvllm_hip.set_option("timing", 0)
    ms_gu, ms_dn = st["ms_gate_up"] / steps, st["ms_down"] / steps
    h2d = st["h2d_weight_bytes"] / steps
    log(f"[{name} T={T} staged] step {wall * 1e6:.1f} us: misses/step "
        f"{st['misses'] / steps:.1f}, hits/step {st['resident_hits'] / steps:.1f}, staged "
        f"{h2d / 2**20:.1f} MiB/step ({h2d / wall / 1e9:.1f} GB/s over the step); gate/up "
        f"{ms_gu * 1e3:.1f} us, down {ms_dn * 1e3:.1f} us (HIP events, compute stream)")
    b_gu, _ = expert_bytes(fmt, D, I)
    gu_gbs = w.nb * b_gu / (ms_gu * 1e-3) / 1e9
    rec = {
        "workload": f"{name} {cfg['desc']}, T={T}, drop-in host entry, {n_miss} of {w.nb} "
                    "experts staged from pinned host memory",
        "value": round(T / wall, 3), "unit": "tokens/s", "ms_per_step": round(wall * 1e3, 6),
        "dtype": "bf16x2", "miss_rate": miss_rate,
        "includes": "PCIe H2D of misses, xg and out; the call's final wait",
        "staged_mib_per_step": round(h2d / 2**20, 2),
        "host_us_per_call": round(st["host_ms"] / steps * 1e3, 1),
        "roofline": {"bound": "hbm", "kernel": "gate_up (resident + staged experts)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    if cpu_seconds > 0:
        rec["cpu_baseline"] = cpu_baseline(np, torch, w, pool, pstride, poff, fmt, D, I, T,
                                           cpu_seconds)
    for b in range(r_res):
        mvllm_hip.evict(0, b)
    L.mvllm_hip_host_free(host)
    del pool
    torch.cuda.empty_cache()
    return rec


def layer_pipeline(np, torch, mvllm_hip, synth, cfg, n_layers=12, steps=4, miss_rate=0.25):
    """The GPU-resident decode of one token through n_layers MoE layers of config c2, the
    HBM tier fed from a pinned RAM tier the way the store feeds it: per layer, routing
    (uniform top-k) picks nb experts, round(miss_rate * nb) of which are not in HBM; they
    are staged with mvllm_hip_prefetch from pinned host blobs, the layer's blob table
    comes from mvllm_hip_tier_table (its stream waits for the copies) and the block runs
    with mvllm_hip_moe_block_routed_dev on segments in device memory.  After each step the
    missed experts are evicted, so every step misses again.
      serialized: layer l's misses staged, then layer l computed, then the host waits
                  (so layer l + 1's copies cannot start during layer l's compute);
      pipelined:  layer l + 1's misses staged while layer l computes (the store's
                  prefetch of the next layer);
      copy only / compute only: the two halves alone.
    Overlap = (serialized - pipelined) / min(copy, compute) per layer."""
    import ctypes
    D, I, fmt, E, k = cfg["D"], cfg["I"], cfg["fmt"], cfg["E"], cfg["k"]
    nbytes, off = mvllm_hip.expert_geom(fmt, D, I)
    stride = (nbytes + 4095) // 4096 * 4096
    rng = np.random.default_rng(77)
    nb = k  # T = 1: one token's k experts
    n_miss = int(round(miss_rate * nb))
    eids = [np.sort(rng.choice(E, size=nb, replace=False)) for _ in range(n_layers)]
    miss = [list(rng.choice(e, size=n_miss, replace=False)) for e in eids]
    # pinned RAM tier: every routed expert of every layer (the resident ones are promoted
    # from it at set-up)
    L = mvllm_hip.lib()
    n_blobs = n_layers * nb
    host = L.mvllm_hip_host_alloc(n_blobs * stride)
    if not host:
        raise SystemExit("pinned host allocation failed")
    pool, _, _, _ = build_pool(torch, mvllm_hip, fmt, D, I, nb, 4321)
    slot = {}
    for l in range(n_layers):
        for j, e in enumerate(eids[l]):
            b = l * nb + j
            slot[(l, int(e))] = host + b * stride
            src = pool[j, :nbytes].cpu().numpy()  # nb distinct blobs, reused across layers
            ctypes.memmove(host + b * stride, src.ctypes.data, nbytes)
    del pool
    torch.cuda.empty_cache()
    for l in range(n_layers):
        for e in eids[l]:
            if e not in miss[l]:
                mvllm_hip.promote(slot[(l, int(e))], nbytes, l, int(e))
    torch.cuda.synchronize()
    # per layer: segments (one token, weights normalized) and x, in device memory
    i32 = dict(dtype=torch.int32, device="cuda")
    segs = []
    for l in range(n_layers):
        w = rng.uniform(0.1, 1.0, nb).astype(np.float32)
        w /= w.sum()
        segs.append((torch.tensor([nb, nb], **i32), torch.tensor(eids[l].astype(np.int32), **i32),
                     torch.arange(nb, **i32), torch.ones(nb, **i32), torch.zeros(nb, **i32),
                     torch.from_numpy(w).cuda()))
    x = torch.from_numpy(rng.standard_normal((1, D)).astype(np.float32)).cuda()
    out = torch.zeros((1, D), dtype=torch.float32, device="cuda")
    table = torch.zeros(E, dtype=torch.int64, device="cuda")

    def stage(l):
        ms = miss[l]
        mvllm_hip.prefetch([l] * len(ms), ms, [slot[(l, int(e))] for e in ms], [nbytes] * len(ms))

    def compute(l):
        mvllm_hip.tier_table(l, E, table)
        c, e_, xo, nr_, rows, rw = segs[l]
        mvllm_hip.moe_block_routed_dev(D, I, fmt, table, E, c, e_, xo, nr_, rows, rw, x, out, 1,
                                       cfg["act"], cfg["a"], cfg["b"])
        mvllm_hip.tier_table_done(l)

    def unstage():
        for l in range(n_layers):
            for e in miss[l]:
                mvllm_hip.evict(l, int(e))

    def run(kind):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        total = 0.0
        for s in range(steps + 1):
            torch.cuda.synchronize()
            e0.record()
            if kind == "pipelined":
                stage(0)
                for l in range(n_layers):
                    compute(l)
                    if l + 1 < n_layers:
                        stage(l + 1)
            else:
                for l in range(n_layers):
                    if kind in ("serialized", "copy"):
                        stage(l)
                    if kind in ("serialized", "compute"):
                        compute(l)
                    if kind == "serialized":  # the next copies start after this compute
                        torch.cuda.synchronize()
            if kind == "copy":  # the copies end on the copy stream: order the end event
                mvllm_hip.tier_table(0, E, table)
            e1.record()
            torch.cuda.synchronize()
            if s > 0:  # the first pass warms up
                total += e0.elapsed_time(e1)
            if kind != "compute":
                unstage()
        return total / steps / n_layers * 1e3  # us per layer

    # compute only: every expert resident
    for l in range(n_layers):
        stage(l)
    torch.cuda.synchronize()
    t_compute = run("compute")
    unstage()
    torch.cuda.synchronize()
    t_copy = run("copy")
    t_ser = run("serialized")
    t_pipe = run("pipelined")
    mvllm_hip.tier_table(0, E, table)
    torch.cuda.synchronize()
    for l in range(n_layers):
        for e in eids[l]:
            mvllm_hip.evict(l, int(e))
    L.mvllm_hip_host_free(host)
    staged_mb = n_miss * nbytes / 1e6
    overlap = (t_ser - t_pipe) / max(min(t_copy, t_compute), 1e-9)
    log(f"layer pipeline c2 ({n_layers} layers, {n_miss} of {nb} experts staged per layer, "
        f"{staged_mb:.1f} MB): per layer copy {t_copy:.1f} us ({staged_mb / t_copy * 1e3:.1f} "
        f"GB/s), compute {t_compute:.1f} us, serialized {t_ser:.1f} us, pipelined "
        f"{t_pipe:.1f} us: overlap {overlap:.2f} of the shorter half")
    return {"workload": f"c2 {cfg['desc']}, T=1, {n_layers} layers, {n_miss} of {nb} experts "
                        "per layer staged from pinned host memory (mvllm_hip_prefetch), blocks "
                        "on device-resident segments (mvllm_hip_moe_block_routed_dev)",
            "us_per_layer": {"copy_only": round(t_copy, 2), "compute_only": round(t_compute, 2),
                             "serialized": round(t_ser, 2), "pipelined": round(t_pipe, 2)},
            "staged_mb_per_layer": round(staged_mb, 2),
            "h2d_gbps": round(staged_mb / t_copy * 1e3, 2),
            "overlap_of_shorter_half": round(overlap, 3),
            "value": round(1e6 / (t_pipe * n_layers), 3), "unit": "tokens/s (12 layers)"}


def cpu_model():
    """The host CPU's model name (reported beside the host baselines)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


@contextlib.contextmanager
def one_core():
    """Pin the process to one of its CPUs while a single-threaded host baseline is timed
    (the reference's host path is single-threaded); yields that CPU's index or None."""
    try:
        old = os.sched_getaffinity(0)
        cpu = min(old)
        os.sched_setaffinity(0, {cpu})
    except (AttributeError, OSError):
        old, cpu = None, None
    try:
        yield cpu
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)


def cpu_baseline(np, torch, w, pool, stride, off, fmt, D, I, T, budget_s):
    """The reference's host moe_block (oracle/_ref build when present, else the C
    restatement) on layer 0's experts, single thread, bounded to ~budget_s.  Decode
    workloads run whole calls (median of at least 5 when they fit the budget); when one
    call would take far longer than the budget (prefill), experts are run one per call (as
    the engine calls moe_block, nb=1) in segment order until the budget is spent, and the
    full call is extrapolated by MACs."""
    import oracle
    kind = "reference" if oracle.have_ref() else "port"
    cpu = oracle.CpuMoe("ref" if kind == "reference" else "oracle")
    from mvllm_hip import synth
    macs_e = [3.0 * D * I * int(n) for n in w.nr]
    macs_total = float(sum(macs_e))

    def expert(i):
        return synth.blob_pieces(pool[i].cpu().numpy(), fmt, D, I, off)

    with one_core() as pinned:
        per, sample = _cpu_time(np, cpu, w, expert, macs_e, macs_total, fmt, D, I, T,
                                budget_s)
    log(f"cpu baseline ({kind}, 1 thread): {per*1e3:.1f} ms/call ({sample})")
    return {"value": round(T / per, 3), "unit": "tokens/s", "cores": 1, "kind": kind,
            "sample": sample, "ms_per_call": round(per * 1e3, 3), "nproc": os.cpu_count(),
            "pinned_cpu": pinned, "cpu_model": cpu_model()}


def _cpu_time(np, cpu, w, expert, macs_e, macs_total, fmt, D, I, T, budget_s):
    """Seconds per moe_block call of the host baseline and a description of the sample."""
    if macs_total / 1e9 <= 4 * budget_s:  # whole calls (about 1 GMAC/s on one core)
        ex = [expert(i) for i in range(w.nb)]
        lists = [[e[k] for e in ex] for k in range(6)]
        ts, t_all = [], time.perf_counter()
        while True:
            o = np.zeros((T, D), np.float32)
            t0 = time.perf_counter()
            cpu.moe_block(w.nb, D, I, fmt, *lists, w.xg, w.xoff, w.nr, w.rows, w.rw, o, T,
                          w.act, w.a, w.b)
            ts.append(time.perf_counter() - t0)
            if (time.perf_counter() - t_all >= budget_s and len(ts) >= 5) or len(ts) >= 50:
                break
        per = float(np.median(ts))
        sample = (f"median of {len(ts)} full moe_block calls of the same workload (T={T}, "
                  f"{w.nb} experts), single-threaded host code")
    else:
        o = np.zeros((T, D), np.float32)
        done, el, n_e = 0.0, 0.0, 0
        for i in range(w.nb):
            g, u, d, gs, us, ds = expert(i)
            j0, n = int(w.xoff[i]), int(w.nr[i])
            t0 = time.perf_counter()
            cpu.moe_block(1, D, I, fmt, [g], [u], [d], [gs], [us], [ds], w.xg[j0:j0 + n],
                          np.zeros(1, np.int32), np.array([n], np.int32), w.rows[j0:j0 + n],
                          w.rw[j0:j0 + n], o, T, w.act, w.a, w.b)
            el += time.perf_counter() - t0
            done += macs_e[i]
            n_e += 1
            if el >= budget_s:
                break
        per = el * macs_total / done
        sample = (f"{n_e} of {w.nb} experts ({int(done / (3 * D * I))} of {int(w.nr.sum())} rows) "
                  f"run as nb=1 calls in {el:.1f} s; the full call extrapolated by MACs")
    return per, sample


if __name__ == "__main__":
    main()
