"""Benchmark of strixite's MTP verify path on one MI355X (BASELINE.json's metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

A step is one MoE FFN verify sublayer: M = 6 tokens, hidden 4096, 512 experts, top-10 routing
from FP32 router logits, SwiGLU experts (gate_up [1024 x 2 x 4096], down [4096 x 1024]) in q4 G = 128. Each step takes
the next of 16 distinct token batches (different routing each, so the 3.4 GB of experts are not served from the
256 MB Infinity Cache), with every input resident in HBM before the timed region. One JSON line goes to stdout:
value = microseconds per layer; roofline = the grouped gate_up + SwiGLU kernel (the dominant one) timed with HIP events
on its stream over a fixed window; cpu_baseline = the CPU oracle's same layer on this host's cores. The line also
carries config 4's prefill tok/s and MFMA fraction and configs 1, 2 and 5 (skip them with --no-extra).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs/layer for q4 MoE verify at M=6 + achieved HBM GB/s; prefill tok/s"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 1_100_000_000  # weight replicas rotated by the dense GEMV lines: > 4x the 256 MB Infinity Cache
TRAFFIC_JSON = os.path.join("profiles", "hbm_traffic.json")
TRAFFIC_GEMV_JSON = os.path.join("profiles", "hbm_traffic_gemv.json")
# configs 1 and 2: (name, bits, N, K, G, M, activation dtype name)
GEMV_CONFIGS = (("cfg1_q4_4096x4096_M1_f32", 4, 4096, 4096, 128, 1, "float32"),
                ("cfg2_q4_12288x4096_M6", 4, 12288, 4096, 128, 6, "bfloat16"),
                ("cfg2_q8_12288x4096_M6", 8, 12288, 4096, 64, 6, "bfloat16"))
COPY_PROBE_BYTES = 256 << 20  # FP32 elements read and written once by the calibration kernel


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip configs 1, 2, 4 (prefill tok/s) and 5")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--probe", action="store_true",
                    help="for rocprofv3 --pmc: a plain copy kernel of known size (the counters' calibration), then the "
                         "config-3 gate_up and down kernels alone, and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only config 4's prefill layer (for rocprofv3 runs): one JSON line with its timings")
    ap.add_argument("--draft-only", action="store_true",
                    help="only the MTP draft head (for rocprofv3 runs): one JSON line with its timings")
    ap.add_argument("--dense-only", action="store_true",
                    help="only the dense prefill-width linears (for rocprofv3 runs): one JSON line with their timings")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only configs 1 and 2, the dense verify-width GEMVs (for rocprofv3 runs): one JSON line")
    ap.add_argument("--tail-only", action="store_true",
                    help="only config 5's verify tail (for rocprofv3 runs): one JSON line with its timings")
    ap.add_argument("--ceilings-only", action="store_true",
                    help="only the streaming-read and MFMA probes (for rocprofv3 runs): one JSON line")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two --probe counter runs (FETCH_SIZE, WRITE_SIZE) into " + TRAFFIC_JSON)
    ap.add_argument("--probe-gemv", action="store_true",
                    help="for rocprofv3 --pmc: the copy kernel, then configs 1 and 2 over their rotated replicas")
    ap.add_argument("--pmc-summary-gemv", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two --probe-gemv counter runs into " + TRAFFIC_GEMV_JSON)
    return ap.parse_args()


def events():
    import torch
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_window(fn, min_launches=400, min_ms=25.0, warm_ms=25.0, windows=5):
    """Milliseconds a launch of fn(i), independent of --steps: launches run for warm_ms (and at least 100) to settle
    the clocks, then `windows` timed windows of at least min_launches launches and min_ms each (HIP events on torch's
    current stream, the stream the kernels run on); the median window's average."""
    import time as _t

    import torch
    i = 0
    t0 = _t.perf_counter()
    while i < 100 or (_t.perf_counter() - t0) * 1e3 < warm_ms:
        fn(i)
        i += 1
        if i % 50 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    per = []
    for _ in range(windows):
        n = min_launches
        while True:
            a, b = events()
            a.record()
            for _j in range(n):
                fn(i)
                i += 1
            b.record()
            b.synchronize()
            ms = a.elapsed_time(b)
            if ms >= min_ms:
                break
            n *= 2
        per.append(ms / n)
    per.sort()
    return per[len(per) // 2]


def gate_up_bytes(U, per_expert, M, d, E, k, I):
    """Algorithmic bytes of one routing + gate_up launch: the U distinct experts' gate_up rows (codes, scales,
    mins), the activations and router logits read, ids / coef and the SwiGLU output written."""
    return U * per_expert + M * d * 2 + M * E * 4 + M * k * (4 + 4) + M * k * I * 2


def down_bytes(U, per_expert, M, d, k, I):
    """Algorithmic bytes of one down + combine launch: the U experts' down rows, h and the routing read, y written."""
    return U * per_expert + M * k * I * 2 + M * k * (4 + 4) + M * d * 2


def moe_layer_bench(args, out):
    import numpy as np
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn
    from strixite_amd.verify import MoeVerifyLayer

    E, d, I, k, M, R = 512, 4096, 1024, 10, 6, 16
    Wr = syn.router_weight(E, d, seed=11)
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=12)
    dn = syn.qweight(4, E * d, I, 128, seed=13)
    xs = [syn.activations(M, d, seed=100 + r) for r in range(R)]
    layer = MoeVerifyLayer(Wr, gu, dn, E, k, M)

    # routing + distinct experts of each batch (untimed)
    per_expert = (gu.nbytes() + dn.nbytes()) // E
    gu_per_expert = gu.nbytes() // E
    Us, bytes_layer, routes = [], [], []
    for r in range(R):
        layer.forward(xs[r])
        ids = layer.ids.clone()
        ws, _ = kx.group_routes(ids, E)
        routes.append((ids, layer.coef.clone(), ws, layer.logits.clone()))
        U = int(torch.unique(ids).numel())
        Us.append(U)
        bytes_layer.append(U * per_expert + Wr.numel() * 4 + 2 * M * d * 2)
    torch.cuda.synchronize()

    # the timed steps: whole layers, rotating the batches. Before the W warm-up steps the layer runs for ~30 ms
    # (untimed) so that the clocks have left their idle state whatever W is.
    t_settle = time.perf_counter()
    i = 0
    while time.perf_counter() - t_settle < 0.03 or i < 64:
        layer.forward(xs[i % R])
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    for i in range(args.warmup):
        layer.forward(xs[i % R])
    torch.cuda.synchronize()
    a, b = events()
    t0 = time.perf_counter()
    a.record()
    for i in range(args.steps):
        layer.forward(xs[i % R])
    b.record()
    b.synchronize()
    wall = time.perf_counter() - t0
    ms_total = a.elapsed_time(b)
    us_layer = ms_total * 1e3 / args.steps
    mean_bytes = sum(bytes_layer[i % R] for i in range(args.steps)) / args.steps
    out["value"] = round(us_layer, 3)
    out["ms_per_step"] = round(ms_total / args.steps, 6)
    out["layer_GBps"] = round(mean_bytes / (us_layer * 1e-6) / 1e9, 1)
    out["layer_hbm_frac"] = round(out["layer_GBps"] / HBM_PEAK_GBS, 4)
    out["distinct_experts_mean"] = round(sum(Us) / R, 2)
    out["wall_s"] = round(wall, 3)

    # dominant kernel alone: routing + gate_up + SwiGLU (the layer's second launch) over the same rotating batches
    h = torch.empty((M, k, I), dtype=torch.bfloat16, device="cuda")
    h_sums = torch.empty((M * k, I // 16), dtype=torch.float32, device="cuda")
    ids_b = torch.empty((M, k), dtype=torch.int32, device="cuda")
    coef_b = torch.empty((M, k), dtype=torch.float32, device="cuda")
    rerr, eerr = torch.zeros(4, dtype=torch.int32, device="cuda"), torch.zeros(4, dtype=torch.int32, device="cuda")
    gsync = kx.verify_layer_sync()  # the pool, as the layer's own launch uses it

    def gate_up(i):
        kx.verify_gate_up(xs[i % R], routes[i % R][3], gu, E, k, ids=ids_b, coef=coef_b, h=h, router_err=rerr,
                          expert_err=eerr, h_sums=h_sums, sync=gsync)

    ms = time_window(gate_up)
    gu_bytes = sum(gate_up_bytes(Us[r], gu_per_expert, M, d, E, k, I) for r in range(R)) / R
    achieved = gu_bytes / (ms * 1e-3) / 1e9
    traffic = None
    tj = os.path.join(ROOT, TRAFFIC_JSON)
    if os.path.exists(tj):  # HBM bytes a launch, measured by rocprofv3 counters (see --probe / --pmc-summary)
        with open(tj) as f:
            traffic = json.load(f).get("gate_up", {}).get("hbm_bytes_per_launch")
    out["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                       "kernel": "gate_up_kernel (routing + gate_up + SwiGLU)", "avg_launch_us": round(ms * 1e3, 3),
                       "algorithmic_bytes_per_launch": int(gu_bytes)}

    # the down projection + combine (the layer's third launch), alone
    hh = [torch.randn((M, k, I), device="cuda").to(torch.bfloat16) for _ in range(R)]
    hs = [t.float().view(M * k, I // 16, 16).sum(-1) for t in hh]  # the 16-feature sums gate_up hands over
    yb = torch.empty((M, d), dtype=torch.bfloat16, device="cuda")
    plans = []  # the routing plan gate_up hands over, one per batch
    for r in range(R):
        plans.append(kx.verify_plan())
        kx.verify_gate_up(xs[r], routes[r][3], gu, E, k, ids=ids_b, coef=coef_b, h=h, router_err=rerr,
                          expert_err=eerr, h_sums=h_sums, plan=plans[r])

    def down(i):
        kx.verify_down(hh[i % R], dn, routes[i % R][0], routes[i % R][1], E, y=yb, expert_err=eerr, h_sums=hs[i % R],
                       plan=plans[i % R])

    ms_dn = time_window(down)
    dn_bytes = sum(down_bytes(Us[r], dn.nbytes() // E, M, d, k, I) for r in range(R)) / R
    out["down_combine"] = {"avg_us": round(ms_dn * 1e3, 3), "GBps": round(dn_bytes / (ms_dn * 1e-3) / 1e9, 1)}

    # the same layer as one launch (sx_moe_verify_layer: projection, routing, gate_up and down as phases of one
    # kernel), over the same rotating batches
    sy = kx.verify_layer_sync()
    lg = torch.empty((M, E), dtype=torch.float32, device="cuda")
    yl = torch.empty((M, d), dtype=torch.bfloat16, device="cuda")

    def one_launch(i):
        kx.verify_layer(xs[i % R], Wr, gu, dn, E, k, sy, logits=lg, ids=ids_b, coef=coef_b, h=h, h_sums=h_sums, y=yl,
                        router_err=rerr, expert_err=eerr)

    ms_one = time_window(one_launch)
    out["one_launch_layer"] = {"avg_us": round(ms_one * 1e3, 3),
                               "GBps": round(mean_bytes / (ms_one * 1e-3) / 1e9, 1)}
    return layer, xs, routes


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(layer, xs, budget_s, gpu_logits):
    """The CPU oracle's same layer (router projection, top-k, SwiGLU experts, combine; FP64 accumulation) on this
    host's cores, over as many of the token batches as fit the time budget, then one batch on a single thread. Also
    counts the tokens whose top-k set differs when routing uses the CPU's own logits instead of the GPU's (near-ties
    of the FP32 projection), over every batch."""
    import numpy as np
    import torch

    from oracle import oracle as orc
    from strixite_amd import synthetic as syn

    E, k, d, I = layer.E, layer.k, layer.d, layer.I
    Wr = layer.Wr.cpu().numpy()
    nproc = os.cpu_count() or 1
    threads = min(nproc, 16)  # the GPU box's CPU share for one GPU, whatever nproc reports
    cache = {}
    prepared = []
    flips = 0
    for r, x in enumerate(xs):
        xh = x.view(torch.int16).cpu().numpy().view(np.uint16)
        logits = orc.linear_f32w(xh, Wr)
        ids, coef, _ = orc.moe_router(logits, E, k)
        g_ids, _, _ = orc.moe_router(gpu_logits[r], E, k)
        flips += int((np.sort(ids, 1) != np.sort(g_ids, 1)).any(1).sum())
        prepared.append((xh, ids))

    def run(r, nthreads):
        xh, ids = prepared[r]
        # the experts the batch touches, copied to the host before the clock starts (resident in RAM on a host)
        touched = [int(e) for e in np.unique(ids)]
        for e in touched:
            if e not in cache:
                cache[e] = (syn.host_rows(layer.gate_up, e * 2 * I, (e + 1) * 2 * I),
                            syn.host_rows(layer.down, e * d, (e + 1) * d))
        remap = {e: i for i, e in enumerate(touched)}
        U = len(touched)
        cat = lambda j, z: np.concatenate([cache[e][j][z] for e in touched])
        hgu = orc.QWeight(4, cat(0, 0), cat(0, 1), cat(0, 2), U * 2 * I, d, 128)
        hdn = orc.QWeight(4, cat(1, 0), cat(1, 1), cat(1, 2), U * d, I, 128)
        t0 = time.perf_counter()
        logits = orc.linear_f32w(xh, Wr, threads=nthreads)
        ids2, coef, _ = orc.moe_router(logits, E, k)
        rid = np.vectorize(remap.get)(ids2).astype(np.int32)
        h, _ = orc.experts_gather(xh, hgu, U, rid, swiglu=True, threads=nthreads)
        orc.experts_combine(h, hdn, U, rid, coef, threads=nthreads)
        return time.perf_counter() - t0

    times = []
    for r in range(len(xs)):
        times.append(run(r, threads))
        if sum(times) >= budget_s:
            break
    t1 = run(0, 1)
    med = sorted(times)[len(times) // 2]
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "single_thread_us": round(t1 * 1e6, 1), "nproc": nproc, "cpu_model": cpu_model(),
            "sample": f"{len(times)} of the {len(xs)} token batches (M = 6 each) through the CPU oracle's layer "
                      f"(median), FP64 accumulation, {threads} threads; single_thread_us: batch 0 on one thread",
            "routing_flips_cpu_vs_gpu_logits": {"tokens": flips, "of": len(xs) * xs[0].shape[0]}}


def prefill_layer(steps=20, probe=False):
    """x BF16 [2048, 4096] through the router projection, the Zipf bias, top-10 routing, grouping,
    the grouped gate_up + SwiGLU and down + combine (q4 G = 128 experts, MFMA 64-slot x 128-row tiles)."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn

    E, d, I, k, M = 512, 4096, 1024, 10, 2048
    Wr = syn.router_weight(E, d, seed=61)
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=62)
    dn = syn.qweight(4, E * d, I, 128, seed=63)
    bias = syn.zipf_router_bias(E, seed=64)
    xs = [syn.activations(M, d, seed=65 + r) for r in range(2)]
    logits = torch.empty((M, E), dtype=torch.float32, device="cuda")
    ids = torch.empty((M, k), dtype=torch.int32, device="cuda")
    coef = torch.empty((M, k), dtype=torch.float32, device="cuda")
    ws = torch.empty(kx.route_workspace_bytes(M, k, E) // 4, dtype=torch.int32, device="cuda")
    h = torch.empty((M, k, I), dtype=torch.bfloat16, device="cuda")
    part = torch.empty((M * k, d), dtype=torch.float32, device="cuda")
    y = torch.empty((M, d), dtype=torch.bfloat16, device="cuda")
    rerr, eerr = torch.zeros(4, dtype=torch.int32, device="cuda"), torch.zeros(4, dtype=torch.int32, device="cuda")
    stamps = {}

    def layer(i, mark=False):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)] if mark else None
        x = xs[i % 2]
        if mark:
            ev[0].record()
        kx.linear_f32w(x, Wr, y=logits)
        logits.add_(bias)
        kx.moe_router(logits, E, k, ids=ids, coef=coef, err=rerr)
        kx.group_routes(ids, E, ws=ws, err=eerr)
        if mark:
            ev[1].record()
        kx.gather_grouped(x, gu, E, ws, M, k, swiglu=True, y=h)
        if mark:
            ev[2].record()
        kx.combine_grouped(h, dn, E, ids, coef, ws, partial=part, y=y)
        if mark:
            ev[3].record()
            stamps[i] = ev

    if probe:  # two layers for rocprofv3 --pmc: the traffic of each kernel a launch
        layer(0)
        layer(1)
        torch.cuda.synchronize()
        U = int((torch.bincount(ids.flatten(), minlength=E) > 0).sum())
        return {"gg_gate_up": U * gu.nbytes() // E + M * d * 2 + M * k * I * 2,
                "gg_down": U * dn.nbytes() // E + M * k * I * 2 + M * d * 2}
    ms = time_window(layer, min_launches=steps, min_ms=30.0, windows=3)
    layer(0, mark=True)
    torch.cuda.synchronize()
    ev = stamps[0]
    t_route, t_gu, t_dn = (ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2]), ev[2].elapsed_time(ev[3]))
    counts = torch.bincount(ids.flatten(), minlength=E)
    U = int((counts > 0).sum())
    flops = 2.0 * M * k * (2 * I * d + d * I)
    wbytes = U * (gu.nbytes() + dn.nbytes()) // E
    return {"us": round(ms * 1e3, 1), "prefill_tok_per_s": round(M / (ms * 1e-3), 1),
            "mfma_frac": round(flops / (ms * 1e-3) / 2.5e15, 4), "expert_weight_GBps": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "routing_us": round(t_route * 1e3, 1), "gate_up_us": round(t_gu * 1e3, 1), "down_combine_us": round(t_dn * 1e3, 1),
            "gate_up_mfma_frac": round(2.0 * M * k * 2 * I * d / (t_gu * 1e-3) / 2.5e15, 4),
            "distinct_experts": U, "max_bucket": int(counts.max()), "flops": flops}


def verify_gemv():
    """Configs 1 and 2: dense q4 / q8 GEMV over weight replicas rotated launch by launch, more than 1.1 GB of them
    (4x the 256 MB Infinity Cache), so every launch reads its weights from HBM."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn

    res = {}
    for name, bits, N, K, G, M, act in GEMV_CONFIGS:
        act = getattr(torch, act)
        one = N * K * bits // 8 + 4 * N * (K // G)
        reps = [syn.qweight(bits, N, K, G, seed=30 + i) for i in range(-(-ROTATE_BYTES // one))]
        x = syn.activations(M, K, seed=40, dtype=act)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        ms = time_window(lambda i: kx.linear(x, reps[i % len(reps)], out_act=0, y=y))
        nbytes = reps[0].nbytes() + x.numel() * x.element_size() + y.numel() * 4
        res[name] = {"us": round(ms * 1e3, 3), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "rotated_MB": round(len(reps) * reps[0].nbytes() / 1e6)}
        del reps
    return res


def extra_configs(out):
    res = verify_gemv()
    # config 4: the MoE layer at prefill width, M = 2048, Zipf-skewed routing; grouped MFMA experts
    res.update(dense_prefill())
    res["cfg4_prefill_layer"] = prefill_layer()
    res["cfg5_verify_tail"] = verify_tail()
    res["mtp_draft_head"] = draft_head()
    out["configs"] = res
    out["ceilings"] = ceilings()


def dense_prefill():
    """Dense linears at prefill width (the route linear_q4_wmma / linear_q8_wmma's callers take): 4096 x 4096 at
    M = 2048 (gg_kernel) and M = 256 (K split over a block's waves, gs_kernel), q4 G = 128 and q8 G = 64, BF16 in
    and out."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn
    res = {}
    for bits, G, seed in ((4, 128, 70), (8, 64, 72)):
        w = syn.qweight(bits, 4096, 4096, G, seed=seed)
        for M in (2048, 256):
            x = syn.activations(M, 4096, seed=seed + 1)
            y = torch.empty((M, 4096), dtype=torch.bfloat16, device="cuda")
            ms = time_window(lambda i: kx.linear(x, w, y=y), min_launches=20, min_ms=20.0)
            res[f"prefill_dense_q{bits}_4096x4096_M{M}"] = {
                "us": round(ms * 1e3, 1), "mfma_frac": round(2.0 * M * 4096 * 4096 / (ms * 1e-3) / 2.5e15, 4)}
            del x, y
        del w
    return res


def ceilings():
    """The part's own ceilings: a streaming read of 1 GiB (4x the Infinity Cache, so every byte comes from HBM) at a few
    grid sizes, and a loop of independent BF16 MFMAs on every SIMD (sx_probe_stream_read, sx_probe_mfma)."""
    import ctypes

    import torch

    import strixite_amd as sx
    L = sx.lib()
    nbytes = 1 << 30
    buf = torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    read = {}
    for blocks in (256, 1024, 4096):
        ms = time_window(lambda i: sx.check(L.sx_probe_stream_read(buf.data_ptr(), nbytes, blocks, sink.data_ptr(), st)),
                         min_launches=20, min_ms=20.0, warm_ms=10.0, windows=3)
        read[f"blocks_{blocks}"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    del buf
    fl = ctypes.c_double()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    mfma = {}
    for per_cu in (2, 4):
        blocks = cus * per_cu
        ms = time_window(lambda i: sx.check(L.sx_probe_mfma(blocks, 4096, sink.data_ptr(), ctypes.byref(fl), st)),
                         min_launches=10, min_ms=20.0, warm_ms=10.0, windows=3)
        mfma[f"waves_per_simd_{per_cu}"] = round(fl.value / (ms * 1e-3) / 1e12, 1)
    return {"stream_read_GBps": read, "stream_read_bytes": nbytes, "stream_read_best_frac": round(
                max(read.values()) / HBM_PEAK_GBS, 4),
            "mfma_bf16_TFLOPs": mfma, "mfma_best_frac": round(max(mfma.values()) / 2500.0, 4)}


def verify_tail(probe=False):
    """Config 5: q8 LM head 151936 x 4096 at M = 6 -> top-40 -> sampled acceptance of 5 drafts."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn
    from strixite_amd.verify import VerifyTail

    V, d = 151936, 4096
    w = syn.qweight(8, V, d, 64, seed=50)
    h = syn.activations(6, d, seed=51)
    tail = VerifyTail(w, V, 40, 6)
    drafts = torch.randint(0, V, (5,), dtype=torch.int32, device="cuda")
    u = torch.rand(6, dtype=torch.float64, device="cuda")
    if probe:  # two verify tails for rocprofv3 --pmc
        for _ in range(2):
            tail.forward(h, drafts, u, 0.7, 40, 0.95)
        torch.cuda.synchronize()
        return {"lm_head": w.nbytes() + h.numel() * 2 + 6 * V * 4}
    ms = time_window(lambda i: tail.forward(h, drafts, u, 0.7, 40, 0.95), min_launches=100, windows=3)
    ms_head = time_window(lambda i: kx.linear(h, w, out_act=0, y=tail.logits[:6]), min_launches=100, windows=3)
    nb = w.nbytes() + h.numel() * 2 + 2 * 6 * V * 4
    return {"us": round(ms * 1e3, 3), "lm_head_us": round(ms_head * 1e3, 3),
            "lm_head_GBps": round((w.nbytes() + 6 * V * 4) / (ms_head * 1e-3) / 1e9, 1),
            "GBps": round(nb / (ms * 1e-3) / 1e9, 1)}


def draft_head():
    """The MTP draft tail at the served shape: the Q4 copy (G = 64) of the first 65,536 rows of a q8 LM head (d = 4096),
    made once on the device, then per draft step h [1, 4096] -> logits [1, 65536] -> top-2 pick."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn
    from strixite_amd.draft import DraftHead

    V, d, mv = 151936, 4096, 65536
    head = syn.qweight(8, V, d, 64, seed=52)
    dh = DraftHead(head, mv)
    # the copy alone (the load-time step; the reference runs it on the host), into the caching allocator's blocks
    copy_ms = time_window(lambda i: kx.quantize_q4_from_q8(head, 64, rows=mv), min_launches=5, min_ms=20.0, warm_ms=5.0,
                          windows=3)
    hs = [syn.activations(1, d, seed=53 + i) for i in range(4)]
    ms = time_window(lambda i: dh.forward(hs[i % 4]), min_launches=200, windows=3)
    nb = dh.w.nbytes() + d * 2 + mv * 4 * 2 + 64
    return {"us": round(ms * 1e3, 3), "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "q4_copy_ms": round(copy_ms, 3),
            "q4_copy_GBps": round((head.q.numel() // V * mv * 1.5 + mv * (d // 64) * 8) / (copy_ms * 1e-3) / 1e9, 1)}


def probe():
    """A plain copy kernel of known size (read COPY_PROBE_BYTES, write COPY_PROBE_BYTES), then the config-3 gate_up
    (routing + gate_up + SwiGLU) and down (+ combine) kernels alone over the rotating batches. Run under rocprofv3
    --pmc FETCH_SIZE (then WRITE_SIZE)."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn
    from strixite_amd.verify import MoeVerifyLayer

    copy_probe()
    E, d, I, k, M, R = 512, 4096, 1024, 10, 6, 16
    Wr = syn.router_weight(E, d, seed=11)
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=12)
    dn = syn.qweight(4, E * d, I, 128, seed=13)
    xs = [syn.activations(M, d, seed=100 + r) for r in range(R)]
    layer = MoeVerifyLayer(Wr, gu, dn, E, k, M)
    routes, Us = [], []
    for r in range(R):
        layer.forward(xs[r])
        routes.append((layer.ids.clone(), layer.coef.clone(), layer.logits.clone()))
        Us.append(int(torch.unique(routes[-1][0]).numel()))
    h = torch.empty((M, k, I), dtype=torch.bfloat16, device="cuda")
    h_sums = torch.empty((M * k, I // 16), dtype=torch.float32, device="cuda")
    ids_b = torch.empty((M, k), dtype=torch.int32, device="cuda")
    coef_b = torch.empty((M, k), dtype=torch.float32, device="cuda")
    yb = torch.empty((M, d), dtype=torch.bfloat16, device="cuda")
    gsync = kx.verify_layer_sync()
    torch.cuda.synchronize()
    for i in range(R):
        kx.verify_gate_up(xs[i], routes[i][2], gu, E, k, ids=ids_b, coef=coef_b, h=h, h_sums=h_sums, sync=gsync)
    for i in range(R):
        kx.verify_down(h, dn, routes[i][0], routes[i][1], E, y=yb, h_sums=h_sums)
    torch.cuda.synchronize()
    alg = {"gate_up": sum(gate_up_bytes(U, gu.nbytes() // E, M, d, E, k, I) for U in Us) / R,
           "down": sum(down_bytes(U, dn.nbytes() // E, M, d, k, I) for U in Us) / R}
    del layer, gu, dn, Wr
    torch.cuda.empty_cache()
    alg.update(prefill_layer(probe=True))  # config 4: grouped gate_up, grouped down (+ its partials' reduce)
    torch.cuda.empty_cache()
    alg.update(verify_tail(probe=True))  # config 5: the q8 LM head, then top-k + acceptance
    print(json.dumps({"probe": "done", "algorithmic_bytes_per_launch": alg, "distinct_experts": Us}))


def copy_probe():
    """The counters' calibration: one elementwise kernel that reads and writes COPY_PROBE_BYTES, five times."""
    import torch
    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.mul(src, 1.0, out=dst)  # one elementwise kernel: reads src, writes dst
    torch.cuda.synchronize()


def probe_gemv():
    """The copy kernel, then configs 1 and 2 each once over all their rotated replicas (every launch a replica not
    read before in the run). Run under rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE)."""
    import torch

    from strixite_amd import kernels as kx
    from strixite_amd import synthetic as syn

    copy_probe()
    alg = {}
    for name, bits, N, K, G, M, act in GEMV_CONFIGS:
        reps = [syn.qweight(bits, N, K, G, seed=30 + i) for i in range(-(-ROTATE_BYTES // (N * K * bits // 8 + 4 * N * (K // G))))]
        x = syn.activations(M, K, seed=40, dtype=getattr(torch, act))
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for w in reps:
            kx.linear(x, w, out_act=0, y=y)
        torch.cuda.synchronize()
        alg[name] = reps[0].nbytes() + x.numel() * x.element_size() + y.numel() * 4
        del reps
        torch.cuda.empty_cache()
    print(json.dumps({"probe": "done", "algorithmic_bytes_per_launch": alg}))


# dense_ks_kernel instantiations of configs 1 and 2 (alone in a --probe-gemv run)
GEMV_KERNELS = (("cfg1_q4_4096x4096_M1_f32", "dense_ks_kernel<4, 3, 4, 1, float, float, false>"),
                ("cfg2_q4_12288x4096_M6", "dense_ks_kernel<4, 1, 4, 1, unsigned short, float, false>"),
                ("cfg2_q8_12288x4096_M6", "dense_ks_kernel<8, 1, 8, 1, unsigned short, float, false>"))


def pmc_summary(fetch_dir, write_dir, gemv=False):
    """Per-launch HBM traffic of the probe's kernels from two rocprofv3 counter runs, each scaled by what the same
    counter reads for the copy kernel (COPY_PROBE_BYTES read and written). gemv: a --probe-gemv run (configs 1 and 2)."""
    import csv
    import glob

    def per_kernel(d, counter):
        rows, copies = {}, []
        for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(fn)):
                if r["Counter_Name"] != counter:
                    continue
                name, v = r["Kernel_Name"], float(r["Counter_Value"]) * 1024.0  # KiB -> bytes
                if "MulFunctor" in name:
                    copies.append((int(r["Grid_Size"]), v))
                if gemv:
                    key = next((k for k, inst in GEMV_KERNELS if inst in name), None)
                else:
                    key = ("gg_down" if "gg_down_kernel" in name else "gg_gate_up" if "gg_kernel" in name
                           else "combine_reduce" if "combine_reduce" in name else "lm_head" if "dense_ks_kernel" in name
                           else "verify_tail" if "topk_accept_kernel" in name else "gate_up" if "gate_up_kernel" in name
                           else "down" if "down_kernel" in name else None)
                if key:
                    rows.setdefault(key, []).append(v)
        big = max(g for g, _ in copies)  # the copy probe: the largest multiply launched
        rows["copy"] = [v for g, v in copies if g == big]
        return {k: sum(v) / len(v) for k, v in rows.items()}

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    f_scale, w_scale = COPY_PROBE_BYTES / fetch["copy"], COPY_PROBE_BYTES / write["copy"]
    out = {"copy_probe_bytes": COPY_PROBE_BYTES, "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
           "note": "FETCH_SIZE / WRITE_SIZE (KiB a dispatch) times the factor that makes the copy kernel read and "
                   "write exactly copy_probe_bytes"}
    keys = [k for k, _ in GEMV_KERNELS] if gemv else ["gate_up", "down", "gg_gate_up", "gg_down", "combine_reduce",
                                                        "lm_head", "verify_tail"]
    for k in keys:
        if k not in fetch or k not in write:
            continue
        fb, wb = fetch[k] * f_scale, write[k] * w_scale
        out[k] = {"fetch_bytes": int(fb), "write_bytes": int(wb), "hbm_bytes_per_launch": int(fb + wb),
                  "raw_fetch_kib": round(fetch[k] / 1024, 1), "raw_write_kib": round(write[k] / 1024, 1)}
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    with open(os.path.join(ROOT, TRAFFIC_GEMV_JSON if gemv else TRAFFIC_JSON), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.pmc_summary_gemv:
        pmc_summary(*args.pmc_summary_gemv, gemv=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported (multi-GPU is a "
                                   "design note only)", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    import strixite_amd
    strixite_amd.lib()  # fails loudly without the built library
    if args.probe:
        probe()
        return
    if args.probe_gemv:
        probe_gemv()
        return
    if args.prefill_only:
        print(json.dumps({"cfg4_prefill_layer": prefill_layer()}))
        return
    if args.draft_only:
        print(json.dumps({"mtp_draft_head": draft_head()}))
        return
    if args.tail_only:
        print(json.dumps({"cfg5_verify_tail": verify_tail()}))
        return
    if args.dense_only:
        print(json.dumps(dense_prefill()))
        return
    if args.gemv_only:
        print(json.dumps(verify_gemv()))
        return
    if args.ceilings_only:
        print(json.dumps({"ceilings": ceilings()}))
        return

    out = {"metric": METRIC, "value": None, "unit": "us/layer", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": None, "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "moe_verify_layer: BASELINE config 3 (M=6, d=4096, E=512, top-10, I=1024, q4 G=128, "
                                  "fp32 router)", "global_batch": 6, "seq_len": 6, "parallelism": "single-gpu"}}
    torch.cuda.synchronize()
    layer, xs, routes = moe_layer_bench(args, out)
    print(f"moe layer: {out['value']} us/layer, {out['layer_GBps']} GB/s; gate_up kernel "
          f"{out['roofline']['achieved']} GB/s", file=sys.stderr, flush=True)
    if not args.no_extra:
        extra_configs(out)
        pf = out["configs"]["cfg4_prefill_layer"]
        out["prefill_tok_per_s"] = pf["prefill_tok_per_s"]
        out["prefill_mfma_frac"] = pf["mfma_frac"]
        print(f"configs: {json.dumps(out['configs'])}", file=sys.stderr, flush=True)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(layer, xs, args.cpu_seconds, [r[3].cpu().numpy() for r in routes])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
