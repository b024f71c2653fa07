"""Benchmark of the MI355X sparse-attention path (BASELINE metric: decode us/layer-step + % HBM roofline at
128K x 4 slots; prefill tok/s at a 2K chunk).

A "step" is one decode layer-step of config C2 (4 slots x 131072 context, k 2048): the SWA ring append, the
compressed-KV and index-key appends, the indexer score over the e4m3 keys, the top-k and the sparse attention over
ring + top-k rows.  Inputs are resident in HBM; NL independent copies of the layer's caches are rotated so every
step misses the 256 MB last-level cache.  The timed region replays a HIP graph of NL layer-steps max(20, K/NL)
times, each replay between two events on the launch stream: the value is the median replay / NL (min, max and the
whole region's mean are reported beside it); `steps` counts the layer-steps the timed region ran (replays x NL).
Each heavy kernel is also replayed alone from a graph of NL launches for its average launch duration (the
roofline denominator).  C4 and C5 are measured the same way and reported under decode_other_configs.

Prints ONE JSON line (rank 0, N = 1)."""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepseekv4.1-a100-custom_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_TFLOPS = 2500.0
MFMA_FP8_TFLOPS = 5000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(cfg, idx_sets=None, fused=True):
    """Algorithmic HBM bytes per launch of the decode kernels.  indexer: per slot the valid index keys (128 B + 4 B
    scale each), per query row the index query and weights and the k indices written; fused (the step's cache
    appends in the same launch): the bf16 index query and weights, and per row the appends' inputs and outputs
    (pre-norm KV row and ring row, latent and compressed row (576 x bf16 each), raw index key (bf16), e4m3 key and
    scale).  sattn: per slot the union of the selected compressed rows and the ring rows (576 x bf16 each), per query
    row q, output and indices."""
    from dsv41_amd.workloads import DQK, DV, H, HI, DI, WIN
    per_kernel = {"indexer": 0, "sattn": 0}
    R = cfg.slots * cfg.rows_per_slot
    for s in range(cfg.slots):
        n = cfg.n_c(s)
        per_kernel["indexer"] += n * (DI + 4)
        sel = min(cfg.topk, n) if idx_sets is None else idx_sets[s]
        per_kernel["sattn"] += (sel + WIN) * DQK * 2
    if fused:
        per_kernel["indexer"] += R * (HI * DI * 2 + HI * 2 + cfg.topk * 4 + 4 * DQK * 2 + DI * 2 + DI + 4)
    else:
        per_kernel["indexer"] += R * (64 * DI + 64 * 4 + cfg.topk * 4)
    per_kernel["sattn"] += R * (H * DQK * 2 + H * DV * 2 + cfg.topk * 4)
    return per_kernel


def step_algorithmic_bytes(cfg, sel_union=None):
    """The per-step algorithmic byte count (keys incl. scale, gathered rows, ring, q, index q, output, idx write +
    read), used for the headline roofline fraction.  Gathered rows per slot: the union of its rows' selections
    (sel_union, measured), or min(k, n) when not given (one row per slot: the same number)."""
    from dsv41_amd.workloads import DQK, DV, H, HI, DI, WIN
    tot = 0
    for s in range(cfg.slots):
        n = cfg.n_c(s)
        r = cfg.rows_per_slot
        rows = min(cfg.topk, n) if sel_union is None else sel_union[s]
        tot += n * (DI + 4) + rows * DQK * 2 + WIN * DQK * 2
        tot += r * (H * DQK * 2 + HI * DI + H * DV * 2 + cfg.topk * 4 * 2)
    return tot


def run_decode(args, dev, name: str, full: bool = True):
    """One decode config: NL cache copies, the layer-step (the step's cache appends + scores + top-k in one launch,
    then the attention; with --separate-appends the appends launch first) captured as a HIP graph of NL layer-steps
    (one per copy).  The graph is replayed max(20, ceil(steps / NL)) times, each replay between two events on the
    launch stream; the value is the median replay / NL, with the min and max.  full: also the eager per-launch
    times (events around each launch) and each heavy kernel alone (a graph of NL launches of it, replayed; its
    average launch duration is the roofline denominator)."""
    import numpy as np
    import torch
    from dsv41_amd.decode import DecodeLayer
    from dsv41_amd.workloads import CONFIGS, make_decode_inputs

    cfg = CONFIGS[name]
    NL = args.layers
    log(f"[bench] building {name}: {cfg.slots} slots x {cfg.rows_per_slot} rows, ctx {cfg.ctx}, {NL} cache copies")
    layers, st = make_decode_inputs(cfg, dev, seed=0, cache_copies=NL)
    rd = 64
    max_pos = max(cfg.ctx) + 8
    ang = torch.outer(torch.arange(max_pos, dtype=torch.float32),
                      1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)))
    cos, sin = torch.cos(ang).to(dev), torch.sin(ang).to(dev)
    L = [DecodeLayer(l["ring"], l["ckv"], l["k8"], l["ks"], st["sink"], cos, sin, cfg.ratio, cfg.topk, rd=rd)
         for l in layers]
    pos, seq, pmax = st["pos"], st["seq"], st["pmax"]
    cl = torch.div(pos + 1, cfg.ratio, rounding_mode="floor")  # once per token, shared by every layer

    fused = not args.separate_appends and cfg.rows_per_slot == 1  # (the fused appends need one row per slot)
    R = cfg.slots * cfg.rows_per_slot

    def appends_select(lay):
        if fused:
            return lay.appends_select(st["kv_raw"], st["kv_norm"], st["latent"], st["k_raw"], st["k_norm"], pos, seq,
                                      st["q_idx"], st["w_idx"], cl)
        lay.appends(st["kv_raw"], st["kv_norm"], st["latent"], st["k_raw"], st["k_norm"], pos, seq, st["q_idx"],
                    st["w_idx"])
        return lay.select(st["q_idx"], st["w_idx"], pos, seq, cl)

    def layer_step(lay):
        idx = appends_select(lay)
        return lay.attend(st["q"], idx, pos, seq, pmax, plim=pos)

    stream = torch.cuda.current_stream(dev)
    for _ in range(max(1, args.warmup)):
        for lay in L:
            layer_step(lay)
    torch.cuda.synchronize(dev)
    E = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    # ---- the selection's union per slot (gathered rows of the attention, for the algorithmic bytes)
    ids = appends_select(L[0]).view(cfg.slots, cfg.rows_per_slot, -1).cpu()
    sel_union = [int(torch.unique(ids[s][ids[s] >= 0]).numel()) for s in range(cfg.slots)]

    # ---- per-phase durations (eager, events around each launch on the launch stream)
    kern_us = {}
    if full:
        phases = {"indexer": [], "sattn": []} if fused else {"appends": [], "indexer": [], "sattn": []}
        for rep in range(max(2, min(args.steps, 20))):
            for lay in L:
                ev = [E() for _ in range(len(phases) + 1)]
                ev[0].record(stream)
                if fused:
                    idx = appends_select(lay)
                else:
                    lay.appends(st["kv_raw"], st["kv_norm"], st["latent"], st["k_raw"], st["k_norm"], pos, seq,
                                st["q_idx"], st["w_idx"])
                    ev[1].record(stream)
                    idx = lay.select(st["q_idx"], st["w_idx"], pos, seq, cl)
                ev[-2].record(stream)
                lay.attend(st["q"], idx, pos, seq, pmax, plim=pos)
                ev[-1].record(stream)
                torch.cuda.synchronize(dev)
                for i, k in enumerate(phases):
                    phases[k].append(ev[i].elapsed_time(ev[i + 1]) * 1000.0)
        kern_us = {k: float(np.median(v)) for k, v in phases.items()}

    # ---- graph of NL layer-steps, replayed; the timed region is bracketed by synchronize
    g = torch.cuda.CUDAGraph()
    s2 = torch.cuda.Stream(dev)
    s2.wait_stream(stream)
    with torch.cuda.stream(s2):
        for lay in L:  # warm the allocator on the capture stream
            layer_step(lay)
    stream.wait_stream(s2)
    torch.cuda.synchronize(dev)
    with torch.cuda.graph(g, stream=s2):
        for lay in L:
            layer_step(lay)
    torch.cuda.synchronize(dev)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize(dev)
    replays = max(20, math.ceil(args.steps / NL))
    ev = [E() for _ in range(replays + 1)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(replays):
        g.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    per = np.array([ev[i].elapsed_time(ev[i + 1]) * 1000.0 / NL for i in range(replays)])
    step_us = float(np.median(per))
    total_us = ev[0].elapsed_time(ev[-1]) * 1000.0 / (replays * NL)
    log(f"[bench] {name} graph: {replays} replays x {NL} layer-steps: median {step_us:.2f} us/layer-step "
        f"(min {per.min():.2f}, max {per.max():.2f}; whole region {total_us:.2f}; wall {wall*1e3:.1f} ms)")
    timing = {"replays": replays, "layer_steps_per_replay": NL, "median_us": round(step_us, 3),
              "min_us": round(float(per.min()), 3), "max_us": round(float(per.max()), 3),
              "region_mean_us": round(total_us, 3)}
    res = dict(cfg=cfg, step_us=step_us, timing=timing, kern_us=kern_us, steps=replays * NL, sel_union=sel_union,
               fused=fused, one_launch=L[0].selector(R, dev).one_launch)
    if not full:
        return res

    # ---- each heavy kernel alone: a graph of NL launches of it (one per cache copy), replayed; the average launch
    # duration (events on the launch stream around the replays) is the roofline denominator
    idxs = [appends_select(lay).clone() for lay in L]
    torch.cuda.synchronize(dev)
    only = {"indexer": lambda lay, i: appends_select(lay) if fused else lay.select(st["q_idx"], st["w_idx"], pos,
                                                                                 seq, cl),
            "sattn": lambda lay, i: lay.attend(st["q"], idxs[i], pos, seq, pmax, plim=pos)}
    alone_us = {}
    for kname, fn in only.items():
        gk = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s2):
            for i, lay in enumerate(L):
                fn(lay, i)
        torch.cuda.synchronize(dev)
        with torch.cuda.graph(gk, stream=s2):
            for i, lay in enumerate(L):
                fn(lay, i)
        gk.replay()
        torch.cuda.synchronize(dev)
        e2, e3 = E(), E()
        e2.record(stream)
        for _ in range(replays):
            gk.replay()
        e3.record(stream)
        torch.cuda.synchronize(dev)
        alone_us[kname] = e2.elapsed_time(e3) * 1000.0 / (replays * NL)
        log(f"[bench] {kname} kernel alone: {alone_us[kname]:.2f} us/launch")
    log(f"[bench] eager per-kernel medians (us): {kern_us}")
    res.update(alone_us=alone_us, kern_bytes=decode_bytes(cfg, sel_union, fused))
    return res


def run_prefill(args, dev):
    """Config C3: one layer's 2048-token chunk after 65536 prior tokens -- the chunk's cache appends (SWA rows,
    compressed rows, index keys), the indexer (score + per-query causal top-2048) and the sparse attention over
    [window history | chunk | compressed] with 128 + 2048 indices per query.  The window and compressed rows are
    read in place (two KV sources) and the selection is written into the compressed columns of one preallocated
    index buffer (the reference concatenates both, dsv41/model.py:1442-1443).  us_per_chunk: a HIP graph of the
    chunk's launches, 5 warm-up replays, then the median of 20 replays each between two events on the launch stream;
    phase_us: eager launches with events between the
    phases, median of the repetitions (the eager appends phase includes host launch time)."""
    import numpy as np
    import torch
    from dsv41_amd import cache as C
    from dsv41_amd.indexer import index_topk
    from dsv41_amd.kernels import sparse_attn
    from dsv41_amd.workloads import PREFILL, make_prefill_inputs, DQK, DV, DI, H, HI, WIN
    cfg = PREFILL["C3"]
    x = make_prefill_inputs(cfg, dev)
    g = torch.Generator(device=dev).manual_seed(7)
    S = cfg.chunk
    kv_raw = (torch.randn(1, S, DQK, generator=g, device=dev)).to(torch.bfloat16)
    kvn = (torch.rand(DQK, generator=g, device=dev) + 0.5).to(torch.bfloat16)
    lat = (torch.randn(1, S // cfg.ratio, DQK, generator=g, device=dev)).to(torch.bfloat16)
    kraw = (torch.randn(1, S // cfg.ratio, DI, generator=g, device=dev)).to(torch.bfloat16)
    kn = (torch.rand(DI, generator=g, device=dev) + 0.5).to(torch.bfloat16)
    ring = torch.zeros(1, WIN, DQK, dtype=torch.bfloat16, device=dev)
    rd = 64
    ang = torch.outer(torch.arange(cfg.end + 8, dtype=torch.float32),
                      1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)))
    cos, sin = torch.cos(ang).to(dev), torch.sin(ang).to(dev)
    ckv_tab = torch.zeros(1, cfg.n_c + 8, DQK, dtype=torch.bfloat16, device=dev)
    ckv_tab[:, :x["ckv"].shape[1]] = x["ckv"]
    kb_tab = torch.zeros(1, cfg.n_c + 8, DI, dtype=torch.bfloat16, device=dev)
    k8_tab = torch.zeros(1, cfg.n_c + 8, DI, dtype=torch.float8_e4m3fn, device=dev)
    ks_tab = torch.zeros(1, cfg.n_c + 8, dtype=torch.float32, device=dev)
    k8_tab[:, :x["k8"].shape[1]] = x["k8"]
    ks_tab[:, :x["ks"].shape[1]] = x["ks"]
    sink = torch.zeros(H, device=dev)
    idx_buf = torch.empty(1, S, WIN + cfg.topk, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    E = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    def step(ev=None):
        if ev: ev[0].record(stream)
        win_kv, widx = C.window_kv(kv_raw, kvn, 1e-6, cos, sin, rd, ring, cfg.prior)
        C.write_compress_kv(ckv_tab, lat, cfg.prior, cfg.ratio, cos, sin, rd)
        C.write_index_k(kb_tab, kraw, kn, 1e-6, cfg.prior, cfg.ratio, cos, sin, rd, k8=k8_tab.view(torch.uint8),
                        k_scale=ks_tab)
        if ev: ev[1].record(stream)
        off = win_kv.shape[1]
        w = widx.shape[-1]
        index_topk(x["q_idx"], x["w_idx"], k8_tab, cfg.prior, cfg.ratio, cfg.topk, off, k_scale=ks_tab,
                   out=idx_buf[:, :, w:w + cfg.topk])
        if ev: ev[2].record(stream)
        idx_buf[:, :, :w].copy_(widx)
        if ev: ev[3].record(stream)
        o = sparse_attn(x["q"], win_kv, sink, idx_buf[:, :, :w + cfg.topk], DQK ** -0.5, d_v=DV,
                        kv2=ckv_tab[:, :cfg.n_c])
        if ev: ev[4].record(stream)
        return o

    for _ in range(2):
        step()
    torch.cuda.synchronize(dev)
    times = {"appends": [], "indexer": [], "glue": [], "attention": [], "total": []}
    for _ in range(max(3, min(args.prefill_reps, 20))):
        ev = [E() for _ in range(5)]
        step(ev)
        torch.cuda.synchronize(dev)
        for i, k in enumerate(["appends", "indexer", "glue", "attention"]):
            times[k].append(ev[i].elapsed_time(ev[i + 1]) * 1000.0)
        times["total"].append(ev[0].elapsed_time(ev[4]) * 1000.0)
    t = {k: float(np.median(v)) for k, v in times.items()}
    # the chunk as a graph of its launches (no host time between them)
    gr = torch.cuda.CUDAGraph()
    s2 = torch.cuda.Stream(dev)
    s2.wait_stream(stream)
    with torch.cuda.stream(s2):
        step()
    torch.cuda.synchronize(dev)
    with torch.cuda.graph(gr, stream=s2):
        step()
    for _ in range(5):  # (warm: the clocks settle over the first replays)
        gr.replay()
    torch.cuda.synchronize(dev)
    reps = 20
    ev = [E() for _ in range(reps + 1)]
    ev[0].record(stream)
    for i in range(reps):
        gr.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize(dev)
    per = np.array([ev[i].elapsed_time(ev[i + 1]) * 1000.0 for i in range(reps)])
    t_graph = float(np.median(per))
    log(f"[bench] prefill C3 graph: median {t_graph:.1f} us/chunk over {reps} replays (min {per.min():.1f}, "
        f"max {per.max():.1f})")
    T = cfg.n_c
    idx_flops = sum(2 * HI * DI * ((cfg.prior + i + 1) // cfg.ratio) for i in range(S))
    att_flops = S * (WIN + cfg.topk) * H * (DQK + DV) * 2
    log(f"[bench] prefill C3 phases (us): {t}")
    return {"config": f"{cfg.name}: {S}-token chunk after {cfg.prior} tokens, ratio {cfg.ratio}, top-k {cfg.topk}, "
                      f"{T} compressed rows, 64 heads x 576",
            "tok_per_s": round(S / (t_graph * 1e-6), 1), "us_per_chunk": round(t_graph, 1),
            "timing": {"replays": reps, "median_us": round(t_graph, 1), "min_us": round(float(per.min()), 1),
                       "max_us": round(float(per.max()), 1)},
            "phase_us": {k: round(v, 1) for k, v in t.items()},
            "mfma_frac": {"indexer_fp8": round(idx_flops / (t["indexer"] * 1e-6) / (MFMA_FP8_TFLOPS * 1e12), 4),
                          "attention_bf16": round(att_flops / (t["attention"] * 1e-6) / (MFMA_BF16_TFLOPS * 1e12), 4),
                          "combined": round((idx_flops / (MFMA_FP8_TFLOPS * 1e12) + att_flops /
                                             (MFMA_BF16_TFLOPS * 1e12)) / (t_graph * 1e-6), 4)}}


# The attention layer's FP8 projections at the reference's decode shapes (results/dense_chain_report.md, table 1:
# dim 5120, q rank 1280, 64 heads x 512, 8 output groups x rank 1024) and its isolated A100 times (us, M = 1).
PROJ_SHAPES = [("wq_a", 1280, 5120, 0, 8.1), ("wq_b", 32768, 1280, 0, 33.4), ("wkv", 512, 5120, 0, 4.9),
               ("wo_a", 8192, 4096, 1024, None), ("wo_b", 5120, 8192, 0, 32.1)]
PRE_MODES = {"wq_b": 1, "wo_b": 2}  # fp8_gemv_m1_pre uses (dsv41/cukern.py:137-158): q_norm before wq_b, quant before wo_b


def run_projections(args, dev):
    """dsv41_fp8_gemm at the projection shapes, M = 1 (the reference's decode) and M = 4 (C2's rows): each weight
    in enough copies to exceed the 256 MB last-level cache, a graph of one launch per copy, replayed; algorithmic
    bytes = weights + scales + x + out."""
    import torch
    from dsv41_amd.w8 import fp8_gemm_tc, fp8_gemv_m1_pre
    res = {}
    for name, N, K, gc, ref_us in PROJ_SHAPES:
        wbytes = N * K + ((N + 31) // 32) * (K // 32)
        copies = max(2, -(-600_000_000 // wbytes))
        ws = []
        for c in range(copies):
            w = torch.randint(0, 256, (N, K), dtype=torch.uint8, device=dev)
            w = torch.where((w & 0x7F) == 0x7F, torch.full_like(w, 0x38), w)
            sc = torch.randint(117, 131, ((N + 31) // 32, K // 32), dtype=torch.uint8, device=dev)
            ws.append((w, sc))
        for M in (1, 4):
            G = N // gc if gc else 1
            x = (torch.randn(M * G, K, device=dev) * 0.1).to(torch.bfloat16)
            s2 = torch.cuda.Stream(dev)
            s2.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(s2):
                for w, sc in ws:
                    fp8_gemm_tc(x, w, sc, gc)
            torch.cuda.synchronize(dev)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=s2):
                for w, sc in ws:
                    fp8_gemm_tc(x, w, sc, gc)
            gr.replay()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            e0.record()
            for _ in range(reps):
                gr.replay()
            e1.record()
            torch.cuda.synchronize(dev)
            us = e0.elapsed_time(e1) * 1000.0 / (reps * copies)
            b = wbytes + M * G * K * 2 + M * N * 2
            gbs = b / (us * 1e-6) / 1e9
            res[f"{name}_M{M}"] = {"N": N, "K": K, "group_cols": gc, "us": round(us, 2), "GB_s": round(gbs, 1),
                                   "hbm_frac": round(gbs / HBM_PEAK_GBS, 3),
                                   "reference_a100_us": ref_us if M == 1 else None}
            log(f"[bench] fp8 projection {name} [{N} x {K}] M={M}: {us:.2f} us, {gbs:.0f} GB/s "
                f"({100 * gbs / HBM_PEAK_GBS:.1f} % of 8 TB/s)")
        if name in PRE_MODES:  # the reference's one-launch GEMV with its activation prologue, one row
            mode = PRE_MODES[name]
            xr = (torch.randn(1, K, device=dev) * 2.0).to(torch.bfloat16)
            nw = (1.0 + 0.1 * torch.randn(K, device=dev)).to(torch.bfloat16)
            s2 = torch.cuda.Stream(dev)
            s2.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(s2):
                for w, sc in ws:
                    fp8_gemv_m1_pre(xr, w, sc, nw, 1e-6, mode)
            torch.cuda.synchronize(dev)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=s2):
                for w, sc in ws:
                    fp8_gemv_m1_pre(xr, w, sc, nw, 1e-6, mode)
            gr.replay()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                gr.replay()
            e1.record()
            torch.cuda.synchronize(dev)
            us = e0.elapsed_time(e1) * 1000.0 / (5 * copies)
            gbs = (wbytes + K * 2 + N * 2) / (us * 1e-6) / 1e9
            res[f"{name}_pre{mode}_M1"] = {"N": N, "K": K, "us": round(us, 2), "GB_s": round(gbs, 1),
                                           "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)}
            log(f"[bench] fp8_gemv_m1_pre mode {mode} {name}: {us:.2f} us")
        del ws
        torch.cuda.empty_cache()
    return res


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    """Threads for the CPU baseline: the job's CPU share (OMP_NUM_THREADS when set, as on the GPU box), else every
    host CPU."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "")))
    except ValueError:
        return os.cpu_count() or 1


def cpu_baseline(cfg, budget_s: float):
    """The reference's PyTorch path on the host in its own precision (oracle/dsv41_torch_cpu.py: the decode indexer's
    bf16 einsum with an fp32 head sum, top-k, and kernels.sparse_attn over ring + selected rows; DSV41_INDEX_BF16=1),
    one whole layer-step of the workload per repetition (every query row of every slot), repeated until the budget
    is spent; the median repetition is the value.  The step's cache appends (a few rows) are left out."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import dsv41_torch_cpu as TC
    from dsv41_amd.workloads import DQK, DV, H, HI, DI, WIN, fp4_round
    torch.set_num_threads(_cpu_threads())
    g = torch.Generator().manual_seed(0)
    S, rps = cfg.slots, cfg.rows_per_slot
    keys = [fp4_round(torch.randn(1, cfg.n_c(s) + 1, DI, generator=g) * 0.1) for s in range(S)]
    ckv = [(torch.randn(1, WIN + cfg.n_c(s) + 1, DQK, generator=g) * 0.1).to(torch.bfloat16) for s in range(S)]
    q = (torch.randn(S, rps, H, DQK, generator=g) * 0.1).to(torch.bfloat16)
    qi = fp4_round(torch.randn(S, rps, HI, DI, generator=g))
    w = (torch.randn(S, rps, HI, generator=g) * (DI ** -0.5 * HI ** -0.5)).to(torch.bfloat16)
    sink = torch.randn(H, generator=g)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or not times:
        t0 = time.perf_counter()
        for s in range(S):
            pos = torch.tensor([cfg.ctx[s] - rps + j for j in range(rps)])
            cl = (pos + 1) // cfg.ratio
            idx = TC.decode_index_topk(qi[s:s + 1].transpose(0, 1), keys[s].expand(rps, -1, -1),
                                       w[s:s + 1].transpose(0, 1), cl, cfg.topk)[:, 0]
            # [ring rows 0..W-1 | compressed rows at W + idx]: the reference's cat of both sources (model.py:1442)
            full = torch.cat([torch.arange(WIN, dtype=torch.int32).expand(rps, -1),
                              torch.where(idx >= 0, idx + WIN, -1)], dim=1)
            TC.sparse_attn(q[s:s + 1], ckv[s], sink, full[None], DQK ** -0.5, dv=DV)
        times.append(time.perf_counter() - t0)
    return {"value": round(float(np.median(times)) * 1e6, 1), "unit": "us/layer-step", "cores": torch.get_num_threads(),
            "host_cpus": os.cpu_count(), "cpu_model": _cpu_model(), "kind": "port",
            "precision": "reference default DSV41_INDEX_BF16=1: bf16 matmuls, fp32 head sum and softmax",
            "sample": f"torch CPU restatement of the reference's decode indexer + kernels.sparse_attn: one whole "
                      f"layer-step of {cfg.name} per repetition ({S * rps} query rows over {S} slots; appends "
                      f"excluded), {len(times)} reps in ~{budget_s:.0f} s, median"}


def cpu_baseline_prefill(budget_s: float, rows: int = 64):
    """The reference's prefill path on the host in its own precision for C3: `rows` query rows of the 2048-token chunk
    (one query chunk of the reference's indexer loop, evenly spaced over the chunk) through the indexer (per-head
    bf16 bmm over the causal compressed keys, fp32 head sum, top-2048; dsv41/model.py:780-893) and kernels.sparse_attn
    over the 128 window + 2048 selected rows, timed and scaled to the chunk: tok/s = 2048 / (time x 2048 / rows)."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import dsv41_torch_cpu as TC
    from dsv41_amd.workloads import DQK, DV, H, HI, DI, WIN, PREFILL, fp4_round
    torch.set_num_threads(_cpu_threads())
    cfg = PREFILL["C3"]
    g = torch.Generator().manual_seed(1)
    T = cfg.n_c
    keys = fp4_round(torch.randn(1, T, DI, generator=g) * 0.1)
    off = WIN - 1 + cfg.chunk
    kv = (torch.randn(1, off + T, DQK, generator=g) * 0.1).to(torch.bfloat16)
    sel = torch.linspace(0, cfg.chunk - 1, rows).long()
    qi = fp4_round(torch.randn(1, cfg.chunk, HI, DI, generator=g))
    w = (torch.randn(1, cfg.chunk, HI, generator=g) * (DI ** -0.5 * HI ** -0.5)).to(torch.bfloat16)
    q = (torch.randn(1, rows, H, DQK, generator=g) * 0.1).to(torch.bfloat16)
    sink = torch.randn(H, generator=g)
    widx = (sel[:, None] + torch.arange(WIN)[None, :]).to(torch.int32)  # the 127 history rows + the row itself
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or not times:
        t0 = time.perf_counter()
        cidx = TC.prefill_index_topk(qi, w, keys, cfg.prior, cfg.ratio, cfg.topk, off, rows=sel)[0]
        TC.sparse_attn(q, kv, sink, torch.cat([widx, cidx], dim=1)[None], DQK ** -0.5, dv=DV)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times)) * cfg.chunk / rows
    return {"value": round(cfg.chunk / t, 2), "unit": "tok/s", "cores": torch.get_num_threads(),
            "host_cpus": os.cpu_count(), "cpu_model": _cpu_model(), "kind": "port",
            "precision": "reference default DSV41_INDEX_BF16=1: bf16 matmuls, fp32 head sum and softmax",
            "sample": f"torch CPU restatement of the reference's prefill indexer + kernels.sparse_attn: {rows} of the "
                      f"chunk's {cfg.chunk} query rows timed (indexer over their causal keys of {T}, top-{cfg.topk}, "
                      f"attention over {WIN} + {cfg.topk} rows), {len(times)} reps in ~{budget_s:.0f} s, median, "
                      f"scaled to the chunk"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--extra-configs", default="C4,C5",
                    help="decode configs also measured (graph replays only) and reported beside the headline")
    ap.add_argument("--layers", type=int, default=8, help="independent cache copies rotated per step")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-proj", action="store_true", help="skip the FP8 projection GEMVs")
    ap.add_argument("--proj-only", action="store_true", help="only the FP8 projection GEMVs (for profiling)")
    ap.add_argument("--separate-appends", action="store_true",
                    help="decode: the cache appends as their own launch before the indexer (default: one launch)")
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--calib-copy", action="store_true", help="one 64 MiB device copy (rocprof counter calibration)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the C3 prefill leg, its phase times printed as JSON (for profiling; not the bench line)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path shards by slot with no exchange; see the design "
              "notes); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.calib_copy:  # 64 MiB read + 64 MiB written by one elementwise kernel (torch neg)
        a = torch.ones(16 << 20, dtype=torch.float32, device=dev)
        b = torch.neg(a)
        torch.cuda.synchronize(dev)
        del a, b
    if args.prefill_only:
        print(json.dumps({"prefill": run_prefill(args, dev)}), flush=True)
        return
    if args.proj_only:
        print(json.dumps({"projections": run_projections(args, dev)}), flush=True)
        return
    r = run_decode(args, dev, args.config)
    cfg = r["cfg"]
    kb, ku = r["kern_bytes"], r["kern_us"]
    R = cfg.slots * cfg.rows_per_slot
    sel_name = ("index_select_kernel<128, true> (cache appends + scores + top-k, one launch)"
                if r["fused"] and r["one_launch"] else
                "index_select_kernel (scores + top-k, one launch)" if r["one_launch"] else
                ("decode_appends_kernel + " if r["fused"] else "") +
                "score kernel with histogram + select kernels (multi-launch)")
    dec32 = os.environ.get("DSV41_ATTN_DEC32", "1") != "0"  # the library's default kernel choice for few rows
    att_name = ("attn_decode32_kernel<576, 512> (32-head workgroups, 128-key splits merged in-kernel)"
                if R < 16 and dec32 else
                "attn_decode_kernel<576, 512> (16-head workgroups, splits merged in-kernel)" if R < 16 else
                "attn_prefill_ws_kernel<576, 512> + attn_decode_combine_kernel (key splits)")
    kernel_names = {"indexer": sel_name, "sattn": att_name}
    roof = {}
    for name, us in r["alone_us"].items():
        achieved = kb[name] / (us * 1e-6) / 1e9
        traffic = None
        tf = os.path.join(ROOT, "profiles", f"{name}_{cfg.name}_traffic.json")
        if os.path.exists(tf):  # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
            with open(tf) as f:
                traffic = json.load(f).get("bytes_per_launch")
        roof[name] = {"bound": "hbm", "kernel": kernel_names[name], "achieved": round(achieved, 1),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                      "traffic": traffic, "algorithmic_bytes": kb[name], "kernel_us": round(us, 3)}
    dom = max(r["alone_us"], key=r["alone_us"].get)  # the kernel with the longest launch
    alg = step_algorithmic_bytes(cfg)
    frac_step = alg / (r["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS
    extra = {}
    for name in [c for c in args.extra_configs.split(",") if c and c != args.config]:
        torch.cuda.empty_cache()
        e = run_decode(args, dev, name, full=False)
        ab = step_algorithmic_bytes(e["cfg"], e["sel_union"])
        extra[name] = {"us_per_layer_step": round(e["step_us"], 3), "timing": e["timing"],
                       "algorithmic_bytes_per_step": ab,
                       "hbm_roofline_pct": round(100.0 * ab / (e["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                       "gathered_rows_per_slot": e["sel_union"],
                       "workload": f"{name}: {e['cfg'].slots} slots x {e['cfg'].rows_per_slot} query rows, ctx "
                                   f"{e['cfg'].ctx}, top-k {e['cfg'].topk}"}
        del e
    torch.cuda.empty_cache()
    pre = None if args.no_prefill else run_prefill(args, dev)
    proj = None if args.no_proj else run_projections(args, dev)
    cpu = None if args.no_cpu else cpu_baseline(cfg, args.cpu_budget)
    if cpu is not None and pre is not None:
        cpu["prefill"] = cpu_baseline_prefill(args.cpu_budget)
    out = {
        "metric": "attn decode us/layer-step + % HBM roofline @128Kx4 slots; prefill tok/s @2K chunk",
        "value": round(r["step_us"], 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": r["steps"],  # layer-steps in the timed region: the graph replays x their layer-steps
        "steps_requested": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_us"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16+fp8e4m3",
        "data": "synthetic (seeded Gaussian, FP4-grid index keys with x8 outlier channels, e4m3 + per-row scale)",
        "config": {"workload": f"{cfg.name}: decode, 1 layer, {cfg.slots} slots x {cfg.ctx[0]} ctx, ratio "
                               f"{cfg.ratio}, top-k {cfg.topk}, SWA {128}, 64 heads x 576 (V 512)",
                   "cache_copies": args.layers},
        "hbm_roofline_pct": round(100.0 * frac_step, 2),
        "timing": r["timing"],
        "algorithmic_bytes_per_step": alg,
        "eager_launch_us": {k: round(v, 3) for k, v in ku.items()},  # eager, one launch each, host gaps included
        "roofline": roof[dom],
        "roofline_other": {k: v for k, v in roof.items() if k != dom},
        "decode_other_configs": extra,
        "prefill": pre,
        "projections": proj,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
