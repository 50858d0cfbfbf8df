"""Benchmark of the table-search path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one MoE layer of the table path on the config-2 workload of
BASELINE.json (Qwen3-VL-30B-A3B-shaped prefill: N=4096 tokens, hidden 2048
bf16, PCA 2048x128 per modality, C=8192 centroids with cached outputs
8192x2048, router 128 experts top-8, keep_rate 0.6, 70 % near / 30 % outlier
tokens): router top-k softmax -> projection -> nearest centroid -> keep-rate
selection -> gather + combine + residual.  Inputs are resident in HBM before
timing; steps rotate over replicas of the workload totalling > 2x the 256 MB
Infinity Cache so reads come from HBM.

Prints ONE JSON line: tokens/s per MoE layer (value, from replays of one HIP
graph holding four consecutive layers, one tm_table_forward call each), per-stage device times, the average
device time of each stage's C-ABI call (graphs of 32 back-to-back calls timed
with HIP events on the stream the kernels run on), the roofline of the
dominant call (HBM bytes from the committed rocprofv3 PMC summary when
present), the decode (N=32, C=16384, top-4) layer, and the reference path
restated on the host CPU (oracle, numpy fp32) as the CPU baseline, and the
config-5 recompute (grouped SwiGLU expert MLP of the kept tokens' slots plus
the shared experts) in its own "recompute" object.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "tablemoe-sc26_amd"))
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "tests"))  # synth.py: seeded workloads of the BASELINE configs

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "table-search tokens/s per MoE layer (N=4096 prefill, N=32 decode) + HBM GB/s"
N_REPLICAS = 4


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _stage_bytes(cfg, n, n_keep, nn, top_k):
    """Algorithmic HBM bytes of each stage of one layer (bf16 = 2 bytes)."""
    H, d, C, E = cfg["hidden"], cfg["dim"], cfg["n_cent"], cfg["n_experts"]
    n_reuse = n - n_keep
    return {
        "router": n * E * 4 + n * top_k * (4 + 8),
        "project": n * H * 2 + 2 * H * d * 2 + 2 * d * 2 + n * d * 2 + n * 4,
        "search": n * d * 2 + C * d * 2 + C * 4 + n * 4 + n * nn * (4 + 8),
        "keep": n * nn * 4 + n,
        "combine": (n + n_keep * top_k * 4 + n_reuse * nn * (8 + (4 if nn > 1 else 0))
                    + n_reuse * nn * H * 2 + n_keep * top_k * H * 2 + 2 * n * H * 2),
    }


def run_layer_bench(cfg_id, steps, warmup, n=None):
    import torch

    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = torch.device("cuda:0")
    t0 = time.time()
    wl = make_workload(cfg_id, n=n)
    log(f"config {cfg_id}: workload generated in {time.time() - t0:.1f}s")
    cfg = wl.cfg
    base = wl.to(dev)
    reps = [base] + [base.to(dev) for _ in range(N_REPLICAS - 1)]
    for r in reps[1:]:
        for k, v in r.__dict__.items():
            if isinstance(v, torch.Tensor):
                setattr(r, k, v.clone())
    tables = [GlobalTable(r.centroids, r.values, (r.proj_vis, r.bias_vis), (r.proj_txt, r.bias_txt)) for r in reps]
    outs = [torch.empty_like(r.residual) for r in reps]
    topk, nn, kr = cfg["router_top_k"], cfg["n_nearest"], cfg["keep_rate"]
    N = cfg["n"]

    stage_names = ["router", "project", "search", "keep", "combine"]

    def step(i, ev=None):
        r, t, o = reps[i % N_REPLICAS], tables[i % N_REPLICAS], outs[i % N_REPLICAS]
        return t.layer_forward(r.x, r.is_vision, r.logits, r.slot_out, r.residual, router_top_k=topk,
                               n_nearest=nn, keep_rate=kr, out=o, stage_events=ev)["keep"]

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    # 1) timed region: K layers back to back, no instrumentation inside
    ev_all = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    ev_all[0].record()
    for i in range(steps):
        step(i)
    ev_all[1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    device_us = 1000.0 * ev_all[0].elapsed_time(ev_all[1]) / steps
    # 1b) the same layers replayed from one HIP graph holding N_REPLICAS
    #     consecutive layers (one per replica, as a model runs its layers):
    #     identical kernels and work, without host launch cost
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(N_REPLICAS):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(N_REPLICAS):
            step(i)
    tail = None  # the last steps % N_REPLICAS layers, so exactly `steps` layers are timed
    if steps % N_REPLICAS:
        tail = torch.cuda.CUDAGraph()
        with torch.cuda.graph(tail):
            for i in range(steps % N_REPLICAS):
                step(i)
    torch.cuda.synchronize()
    for _ in range(max(1, warmup // N_REPLICAS)):
        graph.replay()
    torch.cuda.synchronize()
    g_steps = steps
    g_ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    t_g = time.perf_counter()
    g_ev[0].record()
    for _ in range(steps // N_REPLICAS):
        graph.replay()
    if tail is not None:
        tail.replay()
    g_ev[1].record()
    torch.cuda.synchronize()
    graph_elapsed = time.perf_counter() - t_g
    graph_device_us = 1000.0 * g_ev[0].elapsed_time(g_ev[1]) / g_steps
    del graph, tail
    # 2) instrumented pass over the same steps: HIP events between the stages
    #    (an event record adds a few microseconds of its own between stages)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(steps)]
    for e in evs:  # create the underlying HIP events first
        for x in e:
            x.record()
    torch.cuda.synchronize()
    for i in range(steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    stage_ms = {s: 0.0 for s in stage_names}
    for e in evs:
        for j, s in enumerate(stage_names):
            stage_ms[s] += e[j].elapsed_time(e[j + 1])
    stage_us = {s: 1000.0 * v / steps for s, v in stage_ms.items()}
    keep = step(0)
    torch.cuda.synchronize()
    n_keep = int(keep.sum().item())
    kernel_us = stage_kernel_times(reps, tables, outs, topk, nn, kr)
    return dict(cfg=cfg, wl=wl, elapsed=elapsed, eager_ms_per_step=1000.0 * elapsed / steps,
                ms_per_step=1000.0 * graph_elapsed / g_steps, graph_device_us=graph_device_us, stage_us=stage_us,
                kernel_us=kernel_us, device_us=device_us, n_keep=n_keep,
                bytes=_stage_bytes(cfg, N, n_keep, nn, topk))


def ranked_layer(n, nn, topk, hidden):
    """tm_table_forward ranks the keep set inside the combine for these shapes."""
    return nn == 1 and n <= 4096 and topk in (6, 8) and hidden <= 2048 and hidden % 8 == 0


def stage_kernel_times(reps, tables, outs, topk, nn, kr, launches=32, replays=3):
    """Average device time of each stage's C-ABI call: `launches` back-to-back
    calls (rotating over the table replicas, so reads stay HBM-cold) captured
    in one HIP graph, replayed `replays` times between two HIP events recorded
    on the stream the kernels run on.  The combine stage is the call the layer
    runs: tm_gather_combine_ranked (keep set ranked in the combine) for top-1
    batches of up to 4096 tokens, tm_gather_combine otherwise."""
    import torch

    n0 = reps[0].x.shape[0]
    ranked = ranked_layer(n0, nn, topk, reps[0].x.shape[1])
    rk = [torch.zeros(n0, dtype=torch.bool, device=reps[0].x.device) for _ in reps]

    def calls(name, i):
        r, t, o = reps[i % len(reps)], tables[i % len(tables)], outs[i % len(outs)]
        b = t._bufs
        n = r.x.shape[0]
        if name == "router":
            t.route(r.logits, topk)
        elif name == "project":
            t.project(r.x, r.is_vision)
        elif name == "search":
            t.search(b["q"][: n * t.dim].view(n, t.dim), nn, b["qn"][:n])
        elif name == "keep":
            t.keep_select(b["dist"][: n * nn].view(n, nn)[:, 0], t.keep_count(n, kr))
        elif ranked:  # the layer's combine: keep set ranked in the same launch
            t.gather_combine_ranked(r.slot_out, b["route_w"][: n * topk].view(n, topk), b["idx"][: n * nn].view(n, nn),
                                    b["dist"][:n], t.keep_count(n, kr), r.residual, o, keep=rk[i % len(rk)])
        else:
            t.gather_combine(b["keep"][:n], r.slot_out, b["route_w"][: n * topk].view(n, topk),
                             b["idx"][: n * nn].view(n, nn), b["dist"][: n * nn].view(n, nn), r.residual, o)

    out = {}
    for name in ("router", "project", "search", "keep", "combine"):
        for i in range(len(tables)):  # allocate the stage's own buffers outside capture
            calls(name, i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(launches):
                calls(name, i)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        out[name] = 1000.0 * e0.elapsed_time(e1) / (replays * launches)
        del g
    return out


def run_recompute_bench(steps, warmup):
    """Config 5 recompute (DeepSeek-VL2-style layer, hidden 2560, 64 routed
    experts top-6 + shared experts, intermediate 1536, N=4096): the kept
    tokens' routed slots through tm_group_slots + tm_grouped_swiglu (written
    in the slot layout the combine reads), and the shared-expert MLP (one
    SwiGLU of intermediate 2 x 1536) over every token.  The keep set and the
    router ids come from the config-5 table layer itself; weights are
    random-init N(0, 0.02) bf16 (no checkpoint offline).  Timed as graph
    replays with HIP events on the calls' stream."""
    import torch

    from table_moe.cache_engine import GlobalTable
    from table_moe.ops import GroupedExperts, expert_swiglu
    from synth import make_workload

    dev = torch.device("cuda:0")
    wl = make_workload(5)
    cfg = wl.cfg
    d = wl.to(dev)
    tbl = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    res = tbl.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, cfg["router_top_k"], 1,
                            cfg["keep_rate"])
    keep, ids = res["keep"].clone(), res["ids"].clone()
    n, h, e, k, inter = cfg["n"], cfg["hidden"], cfg["n_experts"], cfg["router_top_k"], 1536
    shared_inter = 2 * inter
    g = torch.Generator(device=dev).manual_seed(55)
    rnd = lambda *shape: (torch.randn(*shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)  # noqa: E731
    ge = GroupedExperts(rnd(e, inter, h), rnd(e, inter, h), rnd(e, h, inter))
    s1, s3, s2 = rnd(shared_inter, h), rnd(shared_inter, h), rnd(h, shared_inter)
    slot_out = torch.empty(n, k, h, dtype=torch.bfloat16, device=dev)
    shared_out = torch.empty(n, h, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(n * shared_inter * 2, dtype=torch.uint8, device=dev)

    def timed(fn, reps):
        for _ in range(max(1, warmup // 4)):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            fn()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return 1000.0 * e0.elapsed_time(e1) / reps

    reps = max(3, min(steps, 20))
    routed_us = timed(lambda: ge.forward(d.x, ids, keep, slot_out), reps)
    shared_us = timed(lambda: expert_swiglu(d.x, s1, s3, s2, out=shared_out, workspace=ws), reps)
    rows = int(keep.sum().item()) * k
    routed_flops = rows * 6.0 * h * inter
    shared_flops = n * 6.0 * h * shared_inter
    tf = lambda f, us: f / (us * 1e-6) / 1e12  # noqa: E731
    return {
        "workload": "config 5 recompute: N=4096, hidden 2560, 64 routed experts top-6 (kept tokens' slots, keep set "
                    "from the config-5 table layer) + shared experts (SwiGLU intermediate 3072, all tokens), routed "
                    "intermediate 1536, random-init bf16 weights",
        "routed_rows": rows,
        "routed_us": routed_us,
        "routed_tflops": tf(routed_flops, routed_us),
        "routed_mfma_frac": tf(routed_flops, routed_us) / BF16_PEAK_TFLOPS,
        "routed_weight_GBps": 3 * e * h * inter * 2 / (routed_us * 1e-6) / 1e9,
        "shared_us": shared_us,
        "shared_tflops": tf(shared_flops, shared_us),
        "shared_mfma_frac": tf(shared_flops, shared_us) / BF16_PEAK_TFLOPS,
    }


COPY_CAL_BYTES = 256 << 20  # bytes read (and written) by the calibration copy


def copy_calibration(reps=3):
    """A plain device copy pass over COPY_CAL_BYTES, launched `reps` times: under
    `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` its counters give the scale
    from counter KiB to bytes moved (profiles/gather_combine_ranked_config2_traffic.txt)."""
    import torch

    a = torch.empty(COPY_CAL_BYTES // 2, dtype=torch.bfloat16, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        torch.neg(a, out=b)  # one elementwise pass: reads and writes COPY_CAL_BYTES (a distinct kernel name)
    torch.cuda.synchronize()
    del a, b


def traffic_from_profile(kernel_prefix, summary):
    """HBM bytes per launch of `kernel_prefix` from the committed PMC summary
    profiles/<summary> (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each
    scaled by the same counter's reading for the calibration copy), or None
    without a summary."""
    path = REPO / "profiles" / summary
    if not path.exists():
        return None
    vals = {}
    for line in path.read_text().splitlines():
        if "=" in line and not line.lstrip().startswith("#"):
            k, v = line.split("=", 1)
            vals[k.strip()] = v.strip()
    try:
        fetch = float(vals[f"{kernel_prefix}.FETCH_SIZE_KiB"]) * 1024.0 * float(vals["copy.fetch_scale"])
        write = float(vals[f"{kernel_prefix}.WRITE_SIZE_KiB"]) * 1024.0 * float(vals["copy.write_scale"])
    except (KeyError, ValueError):
        return None
    return fetch + write


def cpu_baseline(wl, budget_s=12.0):
    """The reference op sequence restated in numpy fp32 (oracle), on a bounded sample."""
    import numpy as np

    from oracle import tm_oracle as O

    try:
        from threadpoolctl import threadpool_info, threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_info = threadpool_limits = None
    f = lambda t: t.detach().cpu().float().numpy()  # noqa: E731
    cfg = wl.cfg
    n_sample = min(cfg["n"], 1024)
    args = (f(wl.x[:n_sample]), wl.is_vision[:n_sample].cpu().numpy(), (f(wl.proj_vis), f(wl.bias_vis)),
            (f(wl.proj_txt), f(wl.bias_txt)), f(wl.centroids), f(wl.values), f(wl.logits[:n_sample]),
            f(wl.slot_out[:n_sample]), f(wl.residual[:n_sample]), cfg["router_top_k"], cfg["n_nearest"],
            cfg["keep_rate"])
    cores = len(os.sched_getaffinity(0))
    threads = cores
    ctx = threadpool_limits(limits=cores) if threadpool_limits else None
    try:
        O.layer_forward_g_fp32(*args)  # warm-up
        times = []
        t_all = time.perf_counter()
        while time.perf_counter() - t_all < budget_s or len(times) < 3:
            t0 = time.perf_counter()
            O.layer_forward_g_fp32(*args)
            times.append(time.perf_counter() - t0)
            if len(times) >= 50:
                break
        if threadpool_info:
            info = threadpool_info()
            if info:
                threads = max(int(i.get("num_threads", 1)) for i in info)
    finally:
        if ctx is not None:
            ctx.unregister() if hasattr(ctx, "unregister") else None
    med = float(np.median(times))
    return {
        "value": n_sample / med,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n_sample} tokens of the config-2 layer (all C={cfg['n_cent']} centroids), "
                  f"median of {len(times)} runs, numpy fp32, {threads} threads on {cores} host cores",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the table-search path runs on a single device in this build "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from table_moe import _native

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    _native.load()
    torch.cuda.set_device(0)
    log(f"device {torch.cuda.get_device_name(0)}")

    pre = run_layer_bench(2, args.steps, args.warmup)
    log(f"prefill: {pre['ms_per_step'] * 1000:.1f} us/layer (graph), {pre['eager_ms_per_step'] * 1000:.1f} eager, "
        f"stages {json.dumps(pre['stage_us'])}")
    dec = run_layer_bench(3, args.steps, args.warmup, n=32)
    log(f"decode N=32: {dec['ms_per_step'] * 1000:.1f} us/layer (graph), {dec['eager_ms_per_step'] * 1000:.1f} eager, "
        f"stages {json.dumps(dec['stage_us'])}")

    cfg = pre["cfg"]
    N, C, d = cfg["n"], cfg["n_cent"], cfg["dim"]
    st, by, ku = pre["stage_us"], pre["bytes"], pre["kernel_us"]
    log(f"prefill per-call device times (graph of 32 calls): {json.dumps({k: round(v, 2) for k, v in ku.items()})}")
    # dominant kernel (longest average call) and its roofline
    dom = max(ku, key=ku.get)
    ranked = ranked_layer(N, cfg["n_nearest"], cfg["router_top_k"], cfg["hidden"])
    entry = {"combine": "tm_gather_combine_ranked" if ranked else "tm_gather_combine", "project": "tm_project",
             "router": "tm_topk_softmax", "keep": "tm_keep_select", "search": "tm_search_global"}[dom]
    if dom == "search":
        flops = 2.0 * N * C * d
        achieved = flops / (ku[dom] * 1e-6) / 1e12
        roof = {"kernel": entry, "bound": "mfma", "achieved": achieved, "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": achieved / BF16_PEAK_TFLOPS, "traffic": None,
                "algorithmic_per_launch": flops}
    else:
        achieved = by[dom] / (ku[dom] * 1e-6) / 1e9
        roof = {"kernel": entry, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBPS,
                "traffic": (traffic_from_profile("gather_combine_rank", "gather_combine_ranked_config2_traffic.txt")
                            if dom == "combine" and ranked else None),
                "algorithmic_per_launch": by[dom]}
    roof["avg_launch_us"] = ku[dom]

    total_bytes = sum(by.values())
    ds = dec["stage_us"]
    search_tflops = 2.0 * N * C * d / (ku["search"] * 1e-6) / 1e12
    result = {
        "metric": METRIC,
        "value": N / (pre["ms_per_step"] * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "config 2: Qwen3-VL-30B-A3B-shaped single MoE layer, prefill N=4096 (3584 vision + 512 "
                        "text), hidden 2048, PCA 2048x128 per modality, C=8192 centroids, cached outputs "
                        "8192x2048, router 128 experts top-8, top-1 search, keep_rate 0.6, 70% near / 30% outliers",
            "tokens": N, "centroids": C, "pca_dim": d, "hidden": cfg["hidden"], "n_keep": pre["n_keep"],
            "replicas": N_REPLICAS,
        },
        "stages_us": {k: round(v, 2) for k, v in st.items()},
        "calls_us": {k: round(v, 2) for k, v in ku.items()},
        "timing": "ms_per_step: layers replayed from one HIP graph of four consecutive layers (one "
                  "tm_table_forward per replica); eager_ms_per_step: one tm_table_forward call per layer "
                  "from Python",
        "eager_ms_per_step": pre["eager_ms_per_step"],
        "eager_tokens_per_s": N / (pre["eager_ms_per_step"] * 1e-3),
        "layer_device_us": pre["graph_device_us"],
        "layer_hbm_GBps": total_bytes / (pre["graph_device_us"] * 1e-6) / 1e9,
        "search_mfma_tflops": search_tflops,
        "search_mfma_frac": search_tflops / BF16_PEAK_TFLOPS,
        "roofline": roof,
        "decode": {
            "workload": "config 3: N=32 text tokens, C=16384 x 128 bf16, cached outputs 16384x2048, top-4 "
                        "inverse-distance blend, keep_rate 0.6",
            "us_per_layer": dec["ms_per_step"] * 1000.0,
            "eager_us_per_layer": dec["eager_ms_per_step"] * 1000.0,
            "layer_device_us": dec["graph_device_us"],
            "tokens_per_s": 32 / (dec["ms_per_step"] * 1e-3),
            "stages_us": {k: round(v, 2) for k, v in ds.items()},
            "calls_us": {k: round(v, 2) for k, v in dec["kernel_us"].items()},
            "search_hbm_GBps": dec["bytes"]["search"] / (dec["kernel_us"]["search"] * 1e-6) / 1e9,
            "layer_hbm_GBps": sum(dec["bytes"].values()) / (dec["graph_device_us"] * 1e-6) / 1e9,
        },
    }
    rec = run_recompute_bench(args.steps, args.warmup)
    log(f"config 5 recompute: routed {rec['routed_us']:.1f} us ({rec['routed_tflops']:.0f} TFLOP/s), shared "
        f"{rec['shared_us']:.1f} us ({rec['shared_tflops']:.0f} TFLOP/s)")
    result["recompute"] = rec
    copy_calibration()
    if not args.no_cpu:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(pre["wl"])
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
