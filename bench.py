"""Benchmark of the table-search path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--sections LIST] [--no-cpu]

A step is one MoE layer of the table path on the config-2 workload of
BASELINE.json (Qwen3-VL-30B-A3B-shaped prefill: N=4096 tokens, hidden 2048
bf16, PCA 2048x128 per modality, C=8192 centroids with cached outputs
8192x2048, router 128 experts top-8, keep_rate 0.6, 70 % near / 30 % outlier
tokens): router top-k softmax -> projection -> nearest centroid -> keep-rate
selection -> gather + combine + residual.  Inputs are resident in HBM before
timing; steps rotate over replicas of the workload totalling > 2x the 256 MB
Infinity Cache so reads come from HBM.

Prints ONE JSON line: the headline (tokens/s per MoE layer from replays of a
HIP graph of four consecutive layers), the roofline of the layer's dominant
kernel (timed live with HIP events on the stream it runs on), and one object
per other BASELINE configuration:
  decode   config 3 at N = 1, 8 and 32 over 128 table replicas (704 MiB of
           distinct tables, so every search reads HBM)
  config1  the fp32 CPU-reference layer on the GPU
  config4  the 48-layer stack, one graph of 48 layers per keep_rate
  config5  the DeepSeek-VL2-style layer end to end (search, grouped
           recompute of the kept slots, shared experts, combine)
  mode_r   the reference's own per-expert searches at Qwen shapes
and the torch-CPU restatement of the reference's fallback path (oracle/
tm_cpu_ref.py) timed on this host's cores for every configuration.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
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
DECODE_REPLICAS = 128
KEEP_RATES = [0.1, 0.25, 0.5, 0.75, 0.9, 1.0]
SECTIONS = ["prefill", "decode", "config1", "config4", "config5", "mode_r", "cpu"]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------- timing helpers
def graph_of(fn):
    """fn() captured in one HIP graph (after an eager run on a side stream, so
    every buffer it uses exists before capture)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def replay_times_us(g, replays, warm=1):
    """Device time of each of `replays` replays of graph g (HIP events on the
    stream the graph runs on), after `warm` untimed replays."""
    import torch

    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    for a, b in evs:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    return [1000.0 * a.elapsed_time(b) for a, b in evs]


def per_call_us(fn, calls=16, replays=10):
    """Device time of one call of fn: a graph of `calls` back-to-back calls,
    median replay time / calls.  (A graph holding one short call is timed at
    the host's graph-launch rate, ~30 us, not at its device time.)"""
    g = graph_of(lambda: [fn() for _ in range(calls)])
    us = statistics.median(replay_times_us(g, replays)) / calls
    del g
    return us


def _stage_bytes(cfg, n, n_keep, nn, top_k):
    """Algorithmic HBM bytes of each stage of one layer (2-byte data)."""
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


def _tables(reps):
    from table_moe.cache_engine import GlobalTable

    return [GlobalTable(r.centroids, r.values, (r.proj_vis, r.bias_vis), (r.proj_txt, r.bias_txt)) for r in reps]


def _replicas(base, count):
    """`count` copies of a device workload in distinct memory."""
    import torch

    out = [base]
    for _ in range(count - 1):
        kw = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in base.__dict__.items()}
        out.append(type(base)(**kw))
    return out


# --------------------------------------------------------------------------- config 2 (headline)
def run_prefill(steps, warmup):
    import torch

    from synth import make_workload

    dev = torch.device("cuda:0")
    t0 = time.time()
    base = make_workload(2).to(dev)
    log(f"config 2: workload generated in {time.time() - t0:.1f}s")
    cfg = base.cfg
    reps = _replicas(base, N_REPLICAS)
    tables = _tables(reps)
    outs = [torch.empty_like(r.residual) for r in reps]
    topk, nn, kr, N = cfg["router_top_k"], cfg["n_nearest"], cfg["keep_rate"], cfg["n"]

    def step(i, ev=None):
        r, t, o = reps[i % N_REPLICAS], tables[i % N_REPLICAS], outs[i % N_REPLICAS]
        return t.layer_forward(r.x, r.is_vision, r.logits, r.slot_out, r.residual, router_top_k=topk,
                               n_nearest=nn, keep_rate=kr, out=o, stage_events=ev)["keep"]

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    # eager: K layers back to back, one C-ABI call each
    t_start = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    eager_s = time.perf_counter() - t_start
    # the timed region of the contract: exactly K layers replayed from HIP
    # graphs of N_REPLICAS consecutive layers (one per replica)
    graph = graph_of(lambda: [step(i) for i in range(N_REPLICAS)])
    tail = graph_of(lambda: [step(i) for i in range(steps % N_REPLICAS)]) if steps % N_REPLICAS else None
    for _ in range(max(1, warmup // N_REPLICAS)):
        graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    t_g = time.perf_counter()
    ev[0].record()
    for _ in range(steps // N_REPLICAS):
        graph.replay()
    if tail is not None:
        tail.replay()
    ev[1].record()
    torch.cuda.synchronize()
    graph_s = time.perf_counter() - t_g
    graph_device_us = 1000.0 * ev[0].elapsed_time(ev[1]) / steps
    # median over >= 100 layers: 32 individually timed replays of the 4-layer graph
    med_us = statistics.median(replay_times_us(graph, 32)) / N_REPLICAS
    del graph, tail
    # instrumented pass: HIP events between the stages.  A bounded device spin
    # (~10 ms) queued first lets the host enqueue every step before the GPU
    # reaches them, so the stage intervals hold device time, not the host's
    # launch latency.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(min(steps, 32))]
    for e in evs:
        for x in e:
            x.record()
    torch.cuda.synchronize()
    torch.cuda._sleep(25_000_000)
    for i, e in enumerate(evs):
        step(i, e)
    torch.cuda.synchronize()
    names = ["router", "project", "search", "keep", "combine"]
    stage_us = {s: 1000.0 * sum(e[j].elapsed_time(e[j + 1]) for e in evs) / len(evs) for j, s in enumerate(names)}
    keep = step(0)
    torch.cuda.synchronize()
    n_keep = int(keep.sum().item())
    kernel_us = stage_call_times(reps, tables, outs, topk, nn, kr)
    return dict(cfg=cfg, reps=reps, eager_us=1e6 * eager_s / steps, graph_us=1e6 * graph_s / steps,
                graph_device_us=graph_device_us, median_us=med_us, stage_us=stage_us, kernel_us=kernel_us,
                n_keep=n_keep, bytes=_stage_bytes(cfg, N, n_keep, nn, topk))


def ranked_layer(n, nn, topk, hidden):
    """tm_table_forward ranks the keep set inside the combine for these shapes."""
    return nn == 1 and n <= 4096 and topk in (6, 8) and hidden <= 2048 and hidden % 8 == 0


def stage_call_times(reps, tables, outs, topk, nn, kr, launches=32, replays=3):
    """Average device time of each stage's C-ABI call: `launches` back-to-back
    calls (rotating over the table replicas, so reads stay HBM-cold) captured
    in one HIP graph, replayed `replays` times between HIP events on the
    stream the kernels run on.  The combine stage is the call the layer runs:
    tm_gather_combine_ranked for top-1 batches of up to 4096 tokens."""
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
        elif ranked:
            t.gather_combine_ranked(r.slot_out, b["route_w"][: n * topk].view(n, topk), b["idx"][: n * nn].view(n, nn),
                                    b["dist"][:n], t.keep_count(n, kr), r.residual, o, keep=rk[i % len(rk)])
        else:
            t.gather_combine(b["keep"][:n], r.slot_out, b["route_w"][: n * topk].view(n, topk),
                             b["idx"][: n * nn].view(n, nn), b["dist"][: n * nn].view(n, nn), r.residual, o)

    out = {}
    for name in ("router", "project", "search", "keep", "combine"):
        for i in range(len(tables)):
            calls(name, i)
        g = graph_of(lambda: [calls(name, i) for i in range(launches)])
        out[name] = sum(replay_times_us(g, replays)) / (replays * launches)
        del g
    return out


COPY_CAL_BYTES = 256 << 20  # bytes read (and written) by the calibration copy


def copy_calibration(reps=3):
    """A plain device copy pass over COPY_CAL_BYTES, launched `reps` times: under
    `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` its counters give the scale
    from counter KiB to bytes moved."""
    import torch

    a = torch.empty(COPY_CAL_BYTES // 2, dtype=torch.bfloat16, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        torch.neg(a, out=b)  # one elementwise pass: reads and writes COPY_CAL_BYTES (a distinct kernel name)
    torch.cuda.synchronize()
    del a, b


def profile_values(summary):
    """key = value lines of a committed profile summary under profiles/."""
    path = REPO / "profiles" / summary
    vals = {}
    if path.exists():
        for line in path.read_text().splitlines():
            if "=" in line and not line.lstrip().startswith("#"):
                k, v = line.split("=", 1)
                vals[k.strip()] = v.strip()
    return vals


def traffic_from_profile(kernel_prefix, summary):
    """HBM bytes per launch of `kernel_prefix` from the committed PMC summary
    (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each scaled by the same
    counter's reading for the calibration copy), or None without one."""
    vals = profile_values(summary)
    try:
        fetch = float(vals[f"{kernel_prefix}.FETCH_SIZE_KiB"]) * 1024.0 * float(vals["copy.fetch_scale"])
        write = float(vals[f"{kernel_prefix}.WRITE_SIZE_KiB"]) * 1024.0 * float(vals["copy.write_scale"])
    except (KeyError, ValueError):
        return None
    return fetch + write


# --------------------------------------------------------------------------- config 3 (decode)
def eager_us(fn, calls=1024, reps=3):
    """Wall time per call of `calls` back-to-back eager calls (no graph), one
    synchronisation at the end: what a loop calling the entry point once per
    token pays, host work or device time, whichever bounds it."""
    import torch

    fn(0)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for i in range(calls):
            fn(i)
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) / calls * 1e6)
    return statistics.median(ts)


def run_decode(replicas=DECODE_REPLICAS, replays=5):
    """Config 3 at N = 1, 8, 32: one HIP graph of `replicas` consecutive layer
    calls, each on its own table (centroids 4 MiB + norms + packed
    projections + cached outputs, all distinct memory), replayed; per-layer
    time = replay time / replicas."""
    import torch

    from synth import make_workload

    dev = torch.device("cuda:0")
    base = make_workload(3, n=32, device=dev, gen_device=dev)
    cfg = base.cfg
    reps = _replicas(base, replicas)
    tables = _tables(reps)
    res = {}
    for n in (1, 8, 32):
        outs = [torch.empty(n, cfg["hidden"], dtype=torch.bfloat16, device=dev) for _ in reps]

        def layers():
            for r, t, o in zip(reps, tables, outs):
                t.layer_forward(r.x[:n], r.is_vision[:n], r.logits[:n], r.slot_out[:n], r.residual[:n], 8, 4, 0.6,
                                out=o)

        g = graph_of(layers)
        per = [t / replicas for t in replay_times_us(g, replays)]
        del g
        args = [(r.x[:n], r.is_vision[:n], r.logits[:n], r.slot_out[:n], r.residual[:n]) for r in reps]

        def eager_layer(i):
            j = i % len(tables)
            tables[j].layer_forward(*args[j], 8, 4, 0.6, out=outs[j])

        eager = eager_us(eager_layer)
        n_keep = max(1, int(n * 0.6))
        by = _stage_bytes(cfg, n, n_keep, 4, 8)
        layer_bytes = (cfg["n_cent"] * cfg["dim"] * 2 + cfg["n_cent"] * 4 + cfg["hidden"] * cfg["dim"] * 2
                       + n * cfg["hidden"] * 2 + 4 * (n - n_keep) * cfg["hidden"] * 2
                       + n_keep * 8 * cfg["hidden"] * 2 + 2 * n * cfg["hidden"] * 2 + n * 8 * 12)
        us = statistics.median(per)
        res[f"N={n}"] = {
            "tokens": n, "n_keep": n_keep, "us_per_layer_median": us, "us_per_layer_mean": statistics.mean(per),
            "tokens_per_s": n / (us * 1e-6), "algorithmic_bytes": layer_bytes,
            "layer_hbm_GBps": layer_bytes / (us * 1e-6) / 1e9,
            "layer_hbm_frac": layer_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "search_bytes": by["search"] + cfg["hidden"] * cfg["dim"] * 2,
            "eager_us_per_layer": eager,
        }
        log(f"decode N={n}: {us:.2f} us/layer (median of {replays} replays of {replicas} layers); "
            f"eager loop {eager:.2f} us per call")
    # the one-launch decode plan's bounded waits: a wait that ran out leaves
    # undefined rows, so a timing it took part in is not a valid measurement
    wait_errors = sum(t.wait_errors() for t in tables)
    if wait_errors:
        raise RuntimeError(f"decode: {wait_errors} cross-workgroup wait(s) ran out during the timed layers")
    res["wait_errors"] = wait_errors
    del reps, tables
    torch.cuda.empty_cache()
    return {"workload": f"config 3: N in {{1, 8, 32}} text tokens, C=16384 x 128 bf16, cached outputs 16384x2048, "
                        f"top-4 inverse-distance blend, keep_rate 0.6; {replicas} distinct tables rotated "
                        f"(704 MiB, > 2x the 256 MB Infinity Cache), one graph of {replicas} layers",
            **res}


# --------------------------------------------------------------------------- config 1
def run_config1(replays=20):
    import torch

    from synth import make_workload

    dev = torch.device("cuda:0")
    reps = _replicas(make_workload(1).to(dev), 8)
    tables = _tables(reps)
    outs = [torch.empty_like(r.residual) for r in reps]

    def layers():
        for r, t, o in zip(reps, tables, outs):
            t.layer_forward(r.x, r.is_vision, r.logits, r.slot_out, r.residual, 8, 1, 0.6, out=o)

    g = graph_of(layers)
    us = statistics.median(replay_times_us(g, replays)) / len(reps)
    del g
    log(f"config 1 (fp32): {us:.2f} us/layer")
    return {"workload": "config 1: N=256, hidden 2048 fp32, PCA 2048x64, C=1024 fp32, cached outputs 1024x2048 "
                        "fp32, router 128 experts top-8, top-1, keep_rate 0.6 (153 kept)",
            "dtype": "f32", "us_per_layer": us, "tokens_per_s": 256 / (us * 1e-6)}


# --------------------------------------------------------------------------- config 4
def run_config4(replays=3):
    """The 48-layer stack: per keep_rate one HIP graph of the 48 layers in
    sequence (layer l's output is layer l + 1's residual)."""
    import torch

    from synth import make_stack

    dev = torch.device("cuda:0")
    t0 = time.time()
    wls = make_stack(48, device=dev)
    torch.cuda.synchronize()
    log(f"config 4: 48 layers generated in {time.time() - t0:.1f}s")
    tables = _tables(wls)
    outs = [torch.empty_like(w.residual) for w in wls]
    cfg = wls[0].cfg
    n = cfg["n"]
    rows = []
    for kr in KEEP_RATES:
        def stack():
            resid = wls[0].residual
            for w, t, o in zip(wls, tables, outs):
                t.layer_forward(w.x, w.is_vision, w.logits, w.slot_out, resid, 8, 1, kr, out=o)
                resid = o

        g = graph_of(stack)
        us = statistics.median(replay_times_us(g, replays)) / len(wls)
        del g
        n_keep = max(1, int(n * kr))
        by = _stage_bytes(cfg, n, n_keep, 1, 8)
        layer_bytes = sum(by.values())
        rows.append({"keep_rate": kr, "n_keep": n_keep, "us_per_layer": us, "tokens_per_s": n / (us * 1e-6),
                     "algorithmic_bytes_per_layer": layer_bytes, "hbm_GBps": layer_bytes / (us * 1e-6) / 1e9,
                     "hbm_frac": layer_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS})
        log(f"config 4 keep {kr}: {us:.2f} us/layer")
    del wls, tables, outs
    torch.cuda.empty_cache()
    return {"workload": "config 4: 48 independent layers (C=8192 x 128, cached outputs 8192x2048 bf16: 1.61 GB of "
                        "tables), N=2048 tokens per layer run in sequence from one HIP graph of 48 layers",
            "keep_rates": rows}


# --------------------------------------------------------------------------- config 5
def run_config5(replays=10):
    """The DeepSeek-VL2-style layer end to end (GlobalTable.layer_forward_recompute)
    and its parts, each as a replayed HIP graph."""
    import torch

    from synth import make_workload
    from table_moe.ops import GroupedExperts, SharedExperts

    dev = torch.device("cuda:0")
    wl = make_workload(5, with_slot_out=False, device=dev, gen_device=dev)
    cfg = wl.cfg
    n, h, e, k, inter = cfg["n"], cfg["hidden"], cfg["n_experts"], cfg["router_top_k"], 1536
    g = torch.Generator(device=dev).manual_seed(55)
    rnd = lambda *shape: (torch.randn(*shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)  # noqa: E731
    ex = GroupedExperts(rnd(e, inter, h), rnd(e, inter, h), rnd(e, h, inter))
    shared = SharedExperts(rnd(2 * inter, h), rnd(2 * inter, h), rnd(h, 2 * inter))
    tbl = _tables([wl])[0]
    out = torch.empty_like(wl.residual)

    def layer():
        tbl.layer_forward_recompute(wl.x, wl.is_vision, wl.logits, ex, wl.residual, k, 0.6, shared=shared, out=out)

    gl = graph_of(layer)
    layer_us = statistics.median(replay_times_us(gl, replays))
    del gl
    res = tbl.layer_forward_recompute(wl.x, wl.is_vision, wl.logits, ex, wl.residual, k, 0.6, shared=shared, out=out)
    keep, ids = res["keep"].clone(), res["ids"].clone()
    w, idx, dist = res["weights"].clone(), res["idx"].clone(), res["dist"].clone()
    slot = res["slot_out"]
    base = torch.empty_like(wl.residual)
    parts = {
        "search_us": lambda: tbl.layer_search(wl.x, wl.is_vision, wl.logits, k, 1, 0.6),
        "routed_recompute_us": lambda: ex.forward(wl.x, ids, keep, slot),
        "shared_us": lambda: shared.forward(wl.x, out=base, addend=wl.residual),
        "combine_us": lambda: tbl.gather_combine(keep, slot, w, idx, dist, base, out),
    }
    times = {}
    for name, fn in parts.items():  # the short parts as graphs of 8 calls (host launch rate otherwise)
        times[name] = per_call_us(fn, 8 if name in ("search_us", "combine_us") else 1, replays)
    rows = int(keep.sum().item()) * k
    routed_flops = rows * 6.0 * h * inter
    shared_flops = n * 6.0 * h * 2 * inter
    search_flops = 2.0 * n * h * cfg["dim"] + 2.0 * n * cfg["n_cent"] * cfg["dim"]
    total_flops = routed_flops + shared_flops + search_flops
    # The routed GEMMs stream every expert's three weight matrices for ~rows/e
    # rows each (~230 FLOP per weight byte at this shape, below the 312 FLOP/B
    # ridge of the bf16 peak over HBM): their bound is HBM.  Bytes they must
    # move: the weights, the gathered x rows, the intermediate written and
    # read once, the slot rows written.
    routed_bytes = 2.0 * (3 * e * inter * h + rows * h + 2 * rows * inter + rows * h)
    log(f"config 5 layer: {layer_us:.1f} us ({json.dumps({k_: round(v, 1) for k_, v in times.items()})})")
    return {
        "workload": "config 5: N=4096, hidden 2560 bf16, 64 routed experts top-6 (intermediate 1536) + shared experts "
                    "(intermediate 2 x 1536), C=8192 x 128, keep_rate 0.6 (2457 kept tokens: 14742 recomputed slot "
                    "rows), random-init N(0, 0.02) bf16 weights; table search -> grouped recompute (packed expert "
                    "weights) -> gather + combine, the shared experts (packed, folded into the residual) on a "
                    "second stream beside the search and the recompute",
        "us_per_layer": layer_us, "tokens_per_s": n / (layer_us * 1e-6), **times,
        "routed_rows": rows, "routed_tflops": routed_flops / (times["routed_recompute_us"] * 1e-6) / 1e12,
        "routed_mfma_frac": routed_flops / (times["routed_recompute_us"] * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
        "routed_algorithmic_bytes": routed_bytes,
        "routed_hbm_frac": routed_bytes / (times["routed_recompute_us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS,
        "shared_tflops": shared_flops / (times["shared_us"] * 1e-6) / 1e12,
        "shared_mfma_frac": shared_flops / (times["shared_us"] * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
        "layer_tflops": total_flops / (layer_us * 1e-6) / 1e12,
    }


# --------------------------------------------------------------------------- mode R
def run_mode_r(replays=20):
    """The reference's own semantics at Qwen3-VL-30B-A3B shapes:
    search_prefill_offline (N=4096, top-8 of 128 experts, reuse = the slots of
    experts outside the 60 % kept by importance) and the decode bs1 hybrid
    search, as replayed HIP graphs."""
    import torch

    from synth import make_mode_r_manager, make_workload
    from table_moe.cache_engine import VectorSearchEngine
    from table_moe.ops import qwen_topk_softmax
    from table_moe.skip import build_prefill_keep_mask

    dev = torch.device("cuda:0")
    mgr = make_mode_r_manager(dev)
    eng = VectorSearchEngine(mgr)
    wl = make_workload(2, with_slot_out=False, device=dev, gen_device=dev)
    n, k = wl.x.shape[0], 8
    w, sel = qwen_topk_softmax(wl.logits, k)
    attn = torch.rand(n, device=dev)
    compute = build_prefill_keep_mask(sel, w, attn, 128, 0.6)
    reuse = ~compute
    # queries that hit their tables: half the tokens sit near a key of their first routed expert
    kb = mgr.keys_buffer
    near = torch.rand(n, device=dev) < 0.5
    src = kb[sel[:, 0], (~wl.is_vision).long(), torch.randint(0, 256, (n,), device=dev)].float()
    p_v, p_t = mgr.pca["vision"]["proj"].float(), mgr.pca["text"]["proj"].float()
    lift = torch.where(wl.is_vision[:, None], src @ p_v.T, src @ p_t.T) * 4.0
    x = torch.where(near[:, None], (wl.x.float() * 0.2 + lift), wl.x.float()).to(torch.bfloat16)
    reuse_frac = float(reuse.float().mean())

    def prefill():
        eng.search_prefill_offline(0, x, sel, wl.is_vision, reuse)

    prefill_us = per_call_us(prefill, 16, replays)
    hit, _ = eng.search_prefill_offline(0, x, sel, wl.is_vision, reuse)
    q = eng.prefill_query_workspace[:n]
    ho = torch.empty(n, k, dtype=torch.bool, device=dev)
    io = torch.empty(n, k, dtype=torch.long, device=dev)
    gated_us = per_call_us(lambda: eng._search_prefill_offline_into(q, sel, wl.is_vision, reuse, ho, io), 16, replays)
    hit_frac = float(hit.float().sum() / reuse.float().sum())
    # decode bs1 hybrid (keep_k 4 of top-8, full 64-entry online window), 64 calls per graph
    outs = [torch.empty(k, dtype=torch.bool, device=dev), torch.empty(1, dtype=torch.long, device=dev),
            torch.empty(k, dtype=torch.bool, device=dev), torch.empty(k, dtype=torch.long, device=dev),
            torch.empty(k, dtype=torch.long, device=dev)]
    xs = x[:64]

    def decode():
        for i in range(64):
            eng.search_decode_hybrid_bs1_into(xs[i], sel[i], wl.is_vision[i], 4, *outs)

    g = graph_of(decode)
    dec_us = statistics.median(replay_times_us(g, replays)) / 64
    del g
    dec_eager_us = eager_us(lambda i: eng.search_decode_hybrid_bs1_into(xs[i % 64], sel[i % 64],
                                                                        wl.is_vision[i % 64], 4, *outs))
    # the decode step's tail for one token (the slot combine with the online
    # window, offline table and recomputed slots, then the ring write:
    # tm_decode_combine_update), after the hybrid search of that token
    eng.search_decode_hybrid_bs1_into(xs[0], sel[0], wl.is_vision[0], 4, *outs)
    comp_rows = (torch.randn(k, x.shape[1], device=dev) * 0.05).to(torch.bfloat16)
    keep_row = torch.zeros(k, dtype=torch.bool, device=dev)
    keep_row[:4] = True
    out_row = torch.empty(x.shape[1], dtype=torch.bfloat16, device=dev)
    step_us = per_call_us(lambda: mgr.combine_and_update_bs1(xs[0], w[0], sel[0], wl.is_vision[0], keep_row,
                                                             comp_rows, outs[0], outs[1], outs[4], outs[2],
                                                             outs[3], out_row), 16, replays)
    pairs = int(reuse.sum().item())
    table_bytes = 128 * 2 * 256 * 64 * 2
    log(f"mode R: search_prefill_offline {prefill_us:.1f} us (gated search {gated_us:.1f} us, {pairs} pairs), "
        f"decode bs1 hybrid {dec_us:.2f} us (eager loop {dec_eager_us:.2f} us per call), decode step combine + "
        f"ring write {step_us:.2f} us")
    return {
        "workload": "mode R (the reference's per-(expert, modality) tables) at Qwen3-VL-30B-A3B shapes: E=128 x 2 "
                    "modalities x K=256 centroids, d=64, hidden 2048 bf16, N=4096 (3584 vision + 512 text), top-8; "
                    "reuse = slots of experts outside the top 60 % by importance",
        "reuse_frac": reuse_frac, "searched_pairs": pairs, "hit_frac": hit_frac,
        "search_prefill_offline_us": prefill_us, "gated_search_us": gated_us,
        "timing": "graphs of 16 back-to-back calls on the same tables (device time per call); decode: 64 calls per "
                  "graph; *_eager_us: 1024 eager calls, one synchronisation at the end (host wall clock)",
        "gated_pairs_per_s": pairs / (gated_us * 1e-6),
        "gated_table_GBps": table_bytes / (gated_us * 1e-6) / 1e9,
        "search_decode_hybrid_bs1_us": dec_us,
        "search_decode_hybrid_bs1_eager_us": dec_eager_us,
        "decode_combine_update_bs1_us": step_us,
    }


def run_mode_r_layer(layers=24):
    """The mode-R prefill layer (Qwen shapes, N=4096) as a drop-in user gets
    it: the table path of QwenMoeWrapperCached.forward in the unchanged
    hook's op order (cached_layers.py:282-465 -- router, the collected
    buffer's zero-fill, keep mask, offline search, torch.where + .cpu() +
    gather_values, the recomputed slots' and the gathered rows' scatters,
    renormalise, bmm) on this package's entry points, with the routed
    experts' outputs given (synthetic, like slot_out in mode G); and the same
    layer with HybridStorageManager.combine_slots (tm_slot_combine) in place
    of :302 and :437-465.  The hook is timed eagerly (its .cpu() syncs the
    host; wall clock per layer, median); the edited layer eagerly and as a
    graph of 16 layers (device time)."""
    import torch

    from synth import make_mode_r_manager, make_workload
    from table_moe.cache_engine import VectorSearchEngine
    from table_moe.ops import qwen_topk_softmax
    from table_moe.skip import build_prefill_keep_mask, renormalize_surviving_weights

    dev = torch.device("cuda:0")
    mgr = make_mode_r_manager(dev)
    eng = VectorSearchEngine(mgr)
    wl = make_workload(2, with_slot_out=False, device=dev, gen_device=dev)
    n, k, H = wl.x.shape[0], 8, wl.x.shape[1]
    g = torch.Generator(device=dev).manual_seed(21)
    logits = wl.logits.to(torch.bfloat16)  # the gate's output in the model dtype
    attn = torch.rand(n, device=dev, generator=g)
    isv = wl.is_vision
    # half the tokens near a key of their first routed expert, so the search hits
    w0, sel0 = qwen_topk_softmax(logits, k)
    kb = mgr.keys_buffer
    near = torch.rand(n, device=dev, generator=g) < 0.5
    src = kb[sel0[:, 0], (~isv).long(), torch.randint(0, 256, (n,), device=dev, generator=g)].float()
    p_v, p_t = mgr.pca["vision"]["proj"].float(), mgr.pca["text"]["proj"].float()
    lift = torch.where(isv[:, None], src @ p_v.T, src @ p_t.T) * 4.0
    x = torch.where(near[:, None], wl.x.float() * 0.2 + lift, wl.x.float()).to(torch.bfloat16)
    expert_out = (torch.randn(n, k, H, device=dev, generator=g) * 0.05).to(torch.bfloat16)

    def hook_layer():
        w, sel = qwen_topk_softmax(logits, k)  # :282
        collected = torch.zeros((n, k, H), dtype=torch.bfloat16, device=dev)  # :302
        compute = build_prefill_keep_mask(sel, w, attn, 128, 0.6)  # :336
        search = ~compute
        off_hit, off_idx = eng.search_prefill_offline(0, x, sel, isv, search)  # :387
        rows, cols = torch.where(off_hit)  # :345-352 perform_value_fetch
        eids = sel[rows, cols].cpu()
        cids = off_idx[rows, cols].cpu()
        mids = torch.where(isv[rows], 0, 1).cpu()
        vals = mgr.gather_values(eids, mids, cids).to(dev, non_blocking=True)
        c_rows, c_cols = torch.where(compute)  # :400, the expert loop's targets (:437)
        collected[c_rows, c_cols] = expert_out[c_rows, c_cols]
        collected[rows, cols] = vals  # :461
        survivor = compute | off_hit
        ew = renormalize_surviving_weights(w, survivor).to(logits.dtype)  # :462
        return torch.bmm(ew.unsqueeze(1), collected).squeeze(1)  # :463

    out_e = torch.empty(n, H, dtype=torch.bfloat16, device=dev)

    def edited_layer():
        w, sel = qwen_topk_softmax(logits, k)
        compute = build_prefill_keep_mask(sel, w, attn, 128, 0.6)
        off_hit, off_idx = eng.search_prefill_offline(0, x, sel, isv, ~compute)
        return mgr.combine_slots(w, sel, isv, compute, expert_out, off_hit, off_idx, out=out_e)

    def wall_us(fn, reps):
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            times.append((time.perf_counter() - t0) * 1e6)
        return statistics.median(times)

    a = hook_layer()
    b = edited_layer()
    torch.cuda.synchronize()
    # the two orders give the same rows up to the combine's rounding (bmm in
    # bf16 vs one fp32 sum): report the largest difference
    max_diff = float((a.float() - b.float()).abs().max())
    for _ in range(3):
        hook_layer()
        edited_layer()
    hook_us = wall_us(hook_layer, layers)
    edited_us = wall_us(edited_layer, layers)
    edited_dev_us = per_call_us(edited_layer, 16, 10)
    # the hook's table-path torch ops alone (device time): zero-fill, scatters, renormalise + bmm
    w, sel = qwen_topk_softmax(logits, k)
    compute = build_prefill_keep_mask(sel, w, attn, 128, 0.6)
    off_hit, off_idx = eng.search_prefill_offline(0, x, sel, isv, ~compute)
    rows, cols = torch.where(off_hit)
    vals = mgr.gather_values(sel[rows, cols], torch.where(isv[rows], 0, 1), off_idx[rows, cols])
    c_rows, c_cols = torch.where(compute)
    collected = torch.empty((n, k, H), dtype=torch.bfloat16, device=dev)

    def hook_torch():
        collected.zero_()
        collected[c_rows, c_cols] = expert_out[c_rows, c_cols]
        collected[rows, cols] = vals
        ew = renormalize_surviving_weights(w, compute | off_hit).to(logits.dtype)
        return torch.bmm(ew.unsqueeze(1), collected).squeeze(1)

    torch_dev_us = per_call_us(hook_torch, 8, 10)
    combine_dev_us = per_call_us(lambda: mgr.combine_slots(w, sel, isv, compute, expert_out, off_hit, off_idx,
                                                           out=out_e), 16, 10)
    hits = int(off_hit.sum())
    log(f"mode R layer (hook op order) {hook_us:.1f} us wall; edited (tm_slot_combine) {edited_us:.1f} us wall, "
        f"{edited_dev_us:.1f} us device; hook torch ops {torch_dev_us:.1f} us vs combine_slots {combine_dev_us:.1f} us")
    return {
        "workload": "mode R prefill layer, Qwen3-VL-30B-A3B shapes (E=128 x 2 x K=256, d=64, hidden 2048 bf16, "
                    "N=4096, top-8, keep 0.6 by importance), the routed experts' outputs given",
        "hook_us": hook_us,
        "edited_us": edited_us,
        "edited_device_us": edited_dev_us,
        "hook_torch_ops_device_us": torch_dev_us,
        "combine_slots_device_us": combine_dev_us,
        "hook_torch_share": (hook_us - edited_us) / hook_us,
        "offline_hits": hits,
        "max_abs_diff_hook_vs_edited": max_diff,
        "tokens_per_s_hook": n / (hook_us * 1e-6),
        "tokens_per_s_edited": n / (edited_dev_us * 1e-6),
        "timing": "hook: eager, host wall clock per layer (its .cpu() syncs), median of "
                  f"{layers}; edited: eager wall clock, and device time from graphs of 16 layers; torch ops / "
                  "combine_slots: graphs of 8 / 16 calls",
    }


# --------------------------------------------------------------------------- CPU baseline
def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(budget_s=30.0):
    """The torch-CPU restatement of the reference fallback path (oracle/
    tm_cpu_ref.py) on this host's cores, fp32 (the CPU's native precision;
    the model dtype would be slower there), median of >= 10 runs after 2
    warm-ups, per configuration; the config-4 and config-5 entries time a
    bounded sample (stated in each)."""
    import torch

    from oracle import tm_cpu_ref as R
    from synth import make_stack, make_workload

    cores = len(os.sched_getaffinity(0))
    threads = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores) or cores))
    torch.set_num_threads(threads)
    per_config_budget = budget_s / 6

    def timed(fn, min_runs=10):
        for _ in range(2):
            fn()
        ts = []
        t_all = time.perf_counter()
        while len(ts) < min_runs or (time.perf_counter() - t_all < per_config_budget and len(ts) < 50):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), len(ts)

    def f32(wl):
        kw = {k: (v.float() if isinstance(v, torch.Tensor) and v.is_floating_point() else v)
              for k, v in wl.__dict__.items()}
        return type(wl)(**kw)

    def layer(w, nn, kr, shared=None):
        return lambda: R.layer_forward_g(w.x, w.is_vision, (w.proj_vis, w.bias_vis), (w.proj_txt, w.bias_txt),
                                         w.centroids, w.values, w.logits, w.slot_out, w.residual,
                                         w.cfg["router_top_k"], nn, kr, shared)

    out = {}
    w1 = f32(make_workload(1))
    t, runs = timed(layer(w1, 1, 0.6))
    out["config1"] = {"us_per_layer": t * 1e6, "tokens_per_s": 256 / t, "runs": runs, "sample": "full layer"}
    log(f"cpu config 1: {t * 1e6:.0f} us/layer")
    w2 = f32(make_workload(2))
    t, runs = timed(layer(w2, 1, 0.6))
    out["config2"] = {"us_per_layer": t * 1e6, "tokens_per_s": 4096 / t, "runs": runs, "sample": "full layer"}
    log(f"cpu config 2: {t * 1e6:.0f} us/layer")
    del w2
    w3 = f32(make_workload(3, n=32))
    for n in (1, 8, 32):
        wn = type(w3)(**{k: (v[:n] if isinstance(v, torch.Tensor) and v.shape[:1] == (32,) else v)
                         for k, v in w3.__dict__.items()})
        t, runs = timed(layer(wn, 4, 0.6))
        out[f"config3_N{n}"] = {"us_per_layer": t * 1e6, "tokens_per_s": n / t, "runs": runs, "sample": "full layer"}
    log(f"cpu config 3 N=32: {out['config3_N32']['us_per_layer']:.0f} us/layer")
    stack = [f32(w) for w in make_stack(2, device="cpu", gen_device="cpu")]
    rows = []
    for kr in KEEP_RATES:
        t, runs = timed(lambda: [layer(w, 1, kr)() for w in stack])
        rows.append({"keep_rate": kr, "us_per_layer": t * 1e6 / len(stack), "tokens_per_s": 2048 * len(stack) / t,
                     "runs": runs})
    out["config4"] = {"sample": "2 of the 48 layers per keep_rate (every layer does the same work)",
                      "keep_rates": rows}
    log(f"cpu config 4 keep 0.5: {rows[2]['us_per_layer']:.0f} us/layer")
    del stack
    ns = 512
    w5 = f32(make_workload(5, n=ns))
    g = torch.Generator().manual_seed(55)
    e, h, inter = 64, 2560, 1536
    ws = [torch.randn(*s, generator=g) * 0.02 for s in ((e, inter, h), (e, inter, h), (e, h, inter))]
    sh = [torch.randn(*s, generator=g) * 0.02 for s in ((2 * inter, h), (2 * inter, h), (h, 2 * inter))]

    def layer5():
        shared = R.swiglu(w5.x, *sh)
        first = R.layer_forward_g(w5.x, w5.is_vision, (w5.proj_vis, w5.bias_vis), (w5.proj_txt, w5.bias_txt),
                                  w5.centroids, w5.values, w5.logits, w5.slot_out, w5.residual, 6, 1, 0.6, shared)
        R.recompute_slots(w5.x, first["ids"], first["keep"], *ws, w5.slot_out)

    t, runs = timed(layer5)
    out["config5"] = {"us_per_layer_sample": t * 1e6, "tokens_per_s": ns / t, "runs": runs,
                      "sample": f"{ns} of the 4096 tokens: search + combine, per-expert recompute of the kept slots "
                                f"and the shared experts (the per-token work of the full layer)"}
    log(f"cpu config 5 ({ns} tokens): {t * 1e3:.1f} ms")
    return {"threads": threads, "cores": cores, "cpu_model": cpu_model(), "dtype": "f32",
            "op_order": "torch-CPU restatement of the reference fallback (oracle/tm_cpu_ref.py): softmax+topk -> "
                        "addmm projection -> addmm distances + min/topk -> keep count -> fancy-index gather -> "
                        "renormalise -> bmm combine (+ residual)",
            "timing": "median of >= 10 runs after 2 warm-ups", **out}


# --------------------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sections", default=",".join(SECTIONS),
                    help=f"comma-separated subset of {SECTIONS} (the headline config 2 always runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the table-search path runs on a single device in this build "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        return 2
    sections = {s.strip() for s in args.sections.split(",") if s.strip()}
    if args.no_cpu:
        sections.discard("cpu")

    import torch

    from table_moe import _native

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    _native.load()
    torch.cuda.set_device(0)
    log(f"device {torch.cuda.get_device_name(0)}")

    pre = run_prefill(args.steps, args.warmup)
    cfg = pre["cfg"]
    N, C, d = cfg["n"], cfg["n_cent"], cfg["dim"]
    st, by, ku = pre["stage_us"], pre["bytes"], pre["kernel_us"]
    log(f"prefill: {pre['graph_us']:.1f} us/layer (graph, wall), {pre['median_us']:.1f} median device, "
        f"{pre['eager_us']:.1f} eager; calls {json.dumps({k: round(v, 2) for k, v in ku.items()})}")
    # dominant call of the layer (longest average call) and its roofline
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
    search_tflops = 2.0 * N * C * d / (ku["search"] * 1e-6) / 1e12
    result = {
        "metric": METRIC,
        "value": N / (pre["graph_us"] * 1e-6),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["graph_us"] / 1000.0,
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
        "timing": "ms_per_step: exactly `steps` layers replayed from HIP graphs of four consecutive layers (one "
                  "tm_table_forward per table replica), wall clock; layer_us_median: median over 128 layers (32 "
                  "individually timed replays); eager_us_per_layer: one C-ABI call per layer from Python",
        "layer_us_median": pre["median_us"],
        "layer_device_us_mean": pre["graph_device_us"],
        "eager_us_per_layer": pre["eager_us"],
        "stages_us": {k: round(v, 2) for k, v in st.items()},
        "calls_us": {k: round(v, 2) for k, v in ku.items()},
        "layer_hbm_GBps": sum(by.values()) / (pre["median_us"] * 1e-6) / 1e9,
        "search_mfma_tflops": search_tflops,
        "search_mfma_frac": search_tflops / BF16_PEAK_TFLOPS,
        "project_hbm_frac": by["project"] / (ku["project"] * 1e-6) / 1e9 / HBM_PEAK_GBPS,
        "roofline": roof,
    }
    del pre
    torch.cuda.empty_cache()
    runners = {"decode": run_decode, "config1": run_config1, "config4": run_config4, "config5": run_config5,
               "mode_r": run_mode_r}
    for name, fn in runners.items():
        if name in sections:
            result[name] = fn()
            torch.cuda.empty_cache()
    if "mode_r" in sections:
        result["mode_r"]["layer"] = run_mode_r_layer()
        torch.cuda.empty_cache()
    copy_calibration()
    if "cpu" in sections:
        log("timing the CPU baseline")
        cpu = cpu_baselines()
        c2 = cpu["config2"]
        result["cpu_baseline"] = {
            "value": c2["tokens_per_s"], "unit": "tokens/s", "cores": cpu["threads"], "kind": "port",
            "sample": f"config 2 full layer (4096 tokens, all 8192 centroids), torch-CPU fp32 restatement of the "
                      f"reference fallback, median of {c2['runs']} runs after 2 warm-ups, {cpu['threads']} threads on "
                      f"{cpu['cores']} cores ({cpu['cpu_model']})",
        }
        result["cpu"] = cpu
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
