"""moe_block benchmark on one MI355X.

Default workload: config c1 (OLMoE shape, int4-g64, D=2048, I=1024, 64 experts,
top-8, SwiGLU) at T=16 decode tokens.  One step = one mvllm_hip_moe_block_dev call
(gate/up/act GEMV, down GEMV, top-k combine) with weights, activations and output
already resident in HBM.  Every step reads its experts from a different layer of a
>= 4 GiB weight pool, so the 256 MB Infinity Cache cannot serve repeated weights.

Prints ONE JSON line on stdout; details go to stderr.
  python bench.py [--steps K] [--warmup W] [--config c1] [--tokens T] [--mode M]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "micro-vllm_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
FP4_PEAK_TFS = 10100.0
BF16_PEAK_TFS = 2500.0


def traffic_bytes(workload, phase):
    """HBM bytes per launch of the workload's gate/up kernel as measured with rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (profiles/traffic.json, calibrated against a copy of
    known size), or None when that workload has not been measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    for k, v in d.get(workload, {}).items():
        if k.endswith(phase):
            return v.get("bytes")
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_pool(torch, mvllm_hip, fmt, D, I, n_blobs, seed):
    """n_blobs expert blobs in the reference layout, generated on the GPU."""
    nbytes, off = mvllm_hip.expert_geom(fmt, D, I)
    stride = (nbytes + 255) // 256 * 256
    g = torch.Generator(device="cuda").manual_seed(seed)
    pool = torch.randint(0, 256, (n_blobs, stride), dtype=torch.uint8, device="cuda",
                         generator=g)
    gq = 64 if fmt == 4 else 32
    pieces = [(1, I, D), (3, I, D), (5, D, I)]  # scale pieces: (offset index, rows O, K)
    for oi, O, K in pieces:
        ns = O * ((K + gq - 1) // gq)
        o = int(off[oi])
        if fmt == 4:
            s = torch.empty((n_blobs, ns), dtype=torch.float32, device="cuda")
            s.uniform_(0.005, 0.02, generator=g)
            s = s.to(torch.bfloat16).to(torch.float32)  # bf16-valued scales stored as f32
            pool[:, o:o + 4 * ns] = s.view(torch.uint8).view(n_blobs, 4 * ns)
        else:
            pool[:, o:o + ns] = torch.randint(118, 125, (n_blobs, ns), dtype=torch.uint8,
                                              device="cuda", generator=g)
    return pool, stride, off, nbytes


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c1")
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--mode", type=int, default=0)
    ap.add_argument("--opt", action="append", default=[], metavar="KEY=VALUE",
                    help="extra mvllm_hip_set_option settings (e.g. dec_ks=2)")
    ap.add_argument("--fp4act", action="store_true",
                    help="MXFP4 experts: quantize activations, native scaled-FP4 matrix cores")
    ap.add_argument("--pool-gb", type=float, default=4.5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--probe-sizes", action="store_true",
                    help="also time the stream-read probe at launch-sized reads (8 MiB .. "
                         "1 GiB, each repetition at a new offset of the pool, so no read is "
                         "served by the Infinity Cache): the floor one launch of that many "
                         "bytes can reach")
    ap.add_argument("--staged", type=float, default=None, metavar="MISS_RATE",
                    help="drop-in host entry with the HBM expert tier: this fraction of each "
                         "step's experts is not resident and is copied from pinned host "
                         "memory by the call (config c2 uses 0.25)")
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
    D, I, E, k, fmt = cfg["D"], cfg["I"], cfg["E"], cfg["k"], cfg["fmt"]
    mvllm_hip.init(0)
    mvllm_hip.set_option("mode", args.mode)
    mvllm_hip.set_option("fp4act", 1 if args.fp4act else 0)
    for kv in args.opt:
        k, v = kv.split("=", 1)
        if not mvllm_hip.set_option(k, int(v)):
            raise SystemExit(f"option {kv} refused")

    if args.staged is not None:
        return staged(args, np, torch, mvllm_hip, synth, cfg, T)

    w = synth.make_workload(args.config, T=T, with_experts=False)
    nbytes, _ = mvllm_hip.expert_geom(fmt, D, I)
    layers = max(1, int(np.ceil(args.pool_gb * 2**30 / (nbytes * w.nb))))
    n_blobs = layers * w.nb
    log(f"workload {args.config} T={T}: {w.nb} experts, {int(w.nr.sum())} rows, "
        f"{layers} pool layers x {w.nb} blobs of {nbytes/2**20:.2f} MiB "
        f"({n_blobs * nbytes / 2**30:.2f} GiB)")
    pool, stride, off, _ = build_pool(torch, mvllm_hip, fmt, D, I, n_blobs, 1234)
    base = pool.data_ptr()

    def lists(layer):
        ptrs = [[], [], [], [], [], []]  # g, u, d, gs, us, ds
        order = (0, 2, 4, 1, 3, 5)       # geometry offsets: gate_p gate_s up_p up_s down_p down_s
        for i in range(w.nb):
            b = base + (layer * w.nb + i) * stride
            for slot, oi in enumerate(order):
                ptrs[slot].append(b + int(off[oi]))
        return ptrs

    layer_lists = [mvllm_hip.prepare_lists(*lists(l)) for l in range(layers)]
    xg = torch.from_numpy(w.xg).cuda()
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    xoff, nr, rows, rw = w.xoff, w.nr, w.rows, w.rw
    # the same arrays every step: their addresses are looked up once (w keeps them alive)
    addr = [xg.data_ptr()] + [a.ctypes.data for a in (xoff, nr, rows, rw)] + [out.data_ptr()]

    def step(s):
        mvllm_hip.moe_block_dev(w.nb, D, I, fmt, None, None, None, None, None, None, *addr[:5],
                                addr[5], T, w.act, w.a, w.b, prepared=layer_lists[s % layers])

    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()

    # timed region: K steps bracketed by synchronize (torch's stream = the null stream,
    # which the library's kernels run on)
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for s in range(args.steps):
        step(s)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps

    # per-kernel durations: a second pass with the library's HIP events around each
    # phase, recorded on the stream the kernels are launched on
    mvllm_hip.set_option("timing", 1)
    mvllm_hip.stats_reset()
    for s in range(args.steps):
        step(s)
    torch.cuda.synchronize()
    st = mvllm_hip.stats()
    mvllm_hip.set_option("timing", 0)
    ms_gu = st["ms_gate_up"] / args.steps
    ms_dn = st["ms_down"] / args.steps
    ms_cb = st["ms_combine"] / args.steps

    # arithmetic of the path the library picks (mvllm_hip.cpp plan_call): native FP4 when
    # asked for; bf16 activations in the grouped GEMM (some expert > 16 rows); otherwise
    # the decode kernels' f32 split into two bf16 terms
    if args.fp4act and fmt == 7:
        dtype = "mxfp4"
    elif int(w.nr.max()) > 16:
        dtype = "bf16" if args.mode != 1 else "bf16x2"
    else:
        dtype = {0: "bf16x2", 1: "bf16x3", 2: "bf16"}[args.mode]
    gq, sb = (64, 4) if fmt == 4 else (32, 1)
    b_gu = 2 * (I * (D // 2) + I * ((D + gq - 1) // gq) * sb)   # gate + up, one expert
    b_dn = D * (I // 2) + D * ((I + gq - 1) // gq) * sb          # down, one expert
    wbytes = w.nb * (b_gu + b_dn)
    flops = 6.0 * D * I * float(w.nr.sum())
    tok_s = T / (ms_step * 1e-3)
    log(f"step {ms_step*1e3:.1f} us (wall {wall/args.steps*1e6:.1f} us): gate/up "
        f"{ms_gu*1e3:.1f} us, down {ms_dn*1e3:.1f} us, combine {ms_cb*1e3:.1f} us; "
        f"effective weight {wbytes/ms_step/1e6:.0f} GB/s")
    gu_gbs = w.nb * b_gu / (ms_gu * 1e-3) / 1e9
    dn_gbs = w.nb * b_dn / (ms_dn * 1e-3) / 1e9
    log(f"gate/up {gu_gbs:.0f} GB/s, down {dn_gbs:.0f} GB/s")

    # achievable HBM streaming-read rate on this box: coalesced 16-byte loads over the
    # whole pool (>= 4 GiB, beyond the Infinity Cache), after one warm-up pass
    sink = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    probe_bytes = (pool.numel() // 4096) * 4096
    hbm_gbs = probe_bytes / mvllm_hip.membench(0, pool, sink, probe_bytes, 0, 5) / 1e6
    # copy probe (1 GiB read + 1 GiB written): with the read probe, the known byte counts
    # that calibrate the FETCH_SIZE / WRITE_SIZE counters of a profiled run
    copy_bytes = min(1 << 30, probe_bytes)
    dst = torch.empty(copy_bytes, dtype=torch.uint8, device="cuda")
    copy_gbs = 2 * copy_bytes / mvllm_hip.membench(1, pool, dst, copy_bytes, 0, 3) / 1e6
    del dst
    log(f"HBM stream-read probe: {hbm_gbs:.0f} GB/s over {probe_bytes / 2**30:.2f} GiB; "
        f"copy probe {copy_gbs:.0f} GB/s (read + write) over {copy_bytes / 2**30:.2f} GiB")
    sizes = {}
    if args.probe_sizes:
        flat = pool.view(-1)
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

    # the routing in front of the block on the device (moe_topk of every token, then the
    # batched call's segments) for this layer shape, and its host counterpart
    route, scores = route_timing(torch, mvllm_hip, T, E, k)
    log(f"device routing (T={T}, E={E}, k={k}): {route['us_per_call']:.2f} us per call")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(np, torch, w, pool, stride, off, fmt, D, I, T, args.cpu_seconds)
        route["cpu_us_per_call"], route["cpu_kind"] = cpu_route_baseline(np, scores, k)
        log(f"host routing: {route['cpu_us_per_call']:.1f} us per call ({route['cpu_kind']})")

    rec = {
        "metric": "moe_block tokens/s (decode), effective weight GB/s",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded; weights random in the reference layouts, in a "
                f"{n_blobs * nbytes / 2**30:.1f} GiB pool rotated per step)",
        "config": {"workload": f"{args.config} {cfg['desc']}, T={T}", "D": D, "I": I, "E": E,
                   "topk": k, "T": T, "fmt": fmt, "experts_per_step": int(w.nb),
                   "rows": int(w.nr.sum()), "mode": args.mode, "fp4act": bool(args.fp4act),
                   "options": args.opt},
        "weight_gbps": round(wbytes / ms_step / 1e6, 1),
        "hbm_probe_gbps": round(hbm_gbs, 1),
        "hbm_copy_probe_gbps": round(copy_gbs, 1),
        **({"hbm_probe_by_size_mib": sizes} if sizes else {}),
        "mfma_util": round(flops / (ms_step * 1e-3) /
                           ((FP4_PEAK_TFS if dtype == "mxfp4" else BF16_PEAK_TFS) * 1e12), 5),
        "roofline": {"bound": "hbm", "kernel": "gate_up_gemv", "achieved": round(gu_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes(f"{args.config} T={T}", "gate_up"),
                     "bytes_per_launch": int(w.nb * b_gu), "avg_launch_us": round(ms_gu * 1e3, 3)},
        "phases_us": {"gate_up": round(ms_gu * 1e3, 3), "down": round(ms_dn * 1e3, 3),
                      "combine": round(ms_cb * 1e3, 3)},
        "cpu_baseline": cpu,
        "route": route,
    }
    print(json.dumps(rec), flush=True)


def route_timing(torch, mvllm_hip, T, E, k, reps=200):
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
    return rec, (choice.cpu().numpy(), mix.cpu().numpy())


def cpu_route_baseline(np, scores, k, budget_s=2.0):
    """The host routing on the same scores: moe_topk per token (oracle/_ref build when
    present, else the C restatement) and the segments (C restatement), one thread."""
    import oracle
    kind = "reference" if oracle.have_ref() else "port"
    topk = oracle.CpuMoe("ref" if kind == "reference" else "oracle")
    seg = oracle.CpuMoe("oracle")
    choice, mix = scores
    T, E = choice.shape
    idx, wt = np.empty((T, k), np.int32), np.empty((T, k), np.float32)
    calls, t0 = 0, time.perf_counter()
    while True:
        for t in range(T):
            _, idx[t], wt[t] = topk.moe_topk(choice[t], k, mix[t])
        seg.moe_segments(idx, wt, T, k, E)
        calls += 1
        if time.perf_counter() - t0 > budget_s:
            break
    return round((time.perf_counter() - t0) / calls * 1e6, 1), \
        f"{kind}; moe_topk per token through ctypes (~1 us call overhead each), then the segments"


def staged(args, np, torch, mvllm_hip, synth, cfg, T):
    """One step = one drop-in mvllm_hip_moe_block call on host pointers (activations and
    output in host memory, as the engine calls it).  Expert blobs live in one pinned host
    buffer (the ExpertStore slots); most are promoted into the library's HBM tier at set-up,
    the rest are host-only, and each step draws round(miss_rate * nb) of its experts from
    them, so the call copies those blobs in on its copy stream while the resident experts
    compute.  Resident and host-only sets rotate over more than the Infinity Cache holds."""
    import ctypes
    D, I, fmt = cfg["D"], cfg["I"], cfg["fmt"]
    w = synth.make_workload(args.config, T=T, with_experts=False)
    nbytes, off = mvllm_hip.expert_geom(fmt, D, I)
    stride = (nbytes + 4095) // 4096 * 4096
    n_miss = int(round(args.staged * w.nb))
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
    log(f"staged {args.config} T={T}: {w.nb} experts/step ({n_res} resident, {n_miss} misses), "
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

    for s in range(args.warmup):
        step(s)
    mvllm_hip.set_option("timing", 1)
    mvllm_hip.stats_reset()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(args.warmup + s)
    wall = (time.perf_counter() - t0) / args.steps
    st = mvllm_hip.stats()
    mvllm_hip.set_option("timing", 0)
    ms_gu, ms_dn = st["ms_gate_up"] / args.steps, st["ms_down"] / args.steps
    h2d = st["h2d_weight_bytes"] / args.steps
    log(f"step {wall * 1e6:.1f} us: misses/step {st['misses'] / args.steps:.1f}, "
        f"hits/step {st['resident_hits'] / args.steps:.1f}, staged {h2d / 2**20:.1f} MiB/step "
        f"({h2d / wall / 1e9:.1f} GB/s over the step); gate/up {ms_gu * 1e3:.1f} us, "
        f"down {ms_dn * 1e3:.1f} us (HIP events, compute stream)")
    gq, sb = (64, 4) if fmt == 4 else (32, 1)
    b_gu = 2 * (I * (D // 2) + I * ((D + gq - 1) // gq) * sb)
    gu_gbs = w.nb * b_gu / (ms_gu * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(np, torch, w, pool, pstride, poff, fmt, D, I, T, args.cpu_seconds)
    rec = {
        "metric": "moe_block tokens/s (decode), effective weight GB/s",
        "value": round(T / wall, 3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16x2",
        "data": "synthetic (seeded; weights random in the reference layouts, pinned host slots)",
        "config": {"workload": f"{args.config} {cfg['desc']}, T={T}, drop-in host entry, "
                               f"{n_miss} of {w.nb} experts staged from pinned host memory",
                   "D": D, "I": I, "E": cfg["E"], "topk": cfg["k"], "T": T, "fmt": fmt,
                   "miss_rate": args.staged, "includes": "PCIe H2D of misses, xg and out"},
        "staged_mib_per_step": round(h2d / 2**20, 2),
        "roofline": {"bound": "hbm", "kernel": "gate_up (resident + staged experts)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


def cpu_baseline(np, torch, w, pool, stride, off, fmt, D, I, T, budget_s):
    """The reference's host moe_block (oracle/_ref build when present, else the C
    restatement) on layer 0's experts, single thread, bounded to ~budget_s.  Decode
    workloads run whole calls; when one call would take far longer than the budget
    (prefill), experts are run one per call (as the engine calls moe_block, nb=1) in
    segment order until the budget is spent, and the full call is extrapolated by MACs."""
    import oracle
    kind = "reference" if oracle.have_ref() else "port"
    cpu = oracle.CpuMoe("ref" if kind == "reference" else "oracle")
    gq, sb = (64, 4) if fmt == 4 else (32, 1)
    macs_e = [3.0 * D * I * int(n) for n in w.nr]
    macs_total = float(sum(macs_e))

    def expert(i):
        host = pool[i].cpu().numpy()

        def piece(oi, O, K, scale):
            o = int(off[oi])
            if scale:
                n = O * ((K + gq - 1) // gq)
                return host[o:o + n * sb].view(np.float32 if fmt == 4 else np.uint8).reshape(O, -1)
            return host[o:o + O * ((K + 1) // 2)].reshape(O, -1)
        return (piece(0, I, D, False), piece(2, I, D, False), piece(4, D, I, False),
                piece(1, I, D, True), piece(3, I, D, True), piece(5, D, I, True))

    if macs_total / 1e9 <= 4 * budget_s:  # whole calls (about 1 GMAC/s on one core)
        ex = [expert(i) for i in range(w.nb)]
        lists = [[e[k] for e in ex] for k in range(6)]
        calls, t0 = 0, time.perf_counter()
        while True:
            o = np.zeros((T, D), np.float32)
            cpu.moe_block(w.nb, D, I, fmt, *lists, w.xg, w.xoff, w.nr, w.rows, w.rw, o, T,
                          w.act, w.a, w.b)
            calls += 1
            el = time.perf_counter() - t0
            if el >= budget_s or calls >= 50:
                break
        per = el / calls
        sample = (f"{calls} full moe_block calls of the same workload (T={T}, {w.nb} experts) "
                  f"in {el:.1f} s, single-threaded host code")
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
    log(f"cpu baseline ({kind}, 1 thread): {per*1e3:.1f} ms/call ({sample})")
    return {"value": round(T / per, 3), "unit": "tokens/s", "cores": 1, "kind": kind,
            "sample": sample, "ms_per_call": round(per * 1e3, 3), "nproc": os.cpu_count()}


if __name__ == "__main__":
    main()
