"""Benchmark of the MoE expert-layer hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2] [--gpus 1]
                    [--no-cpu-baseline] [--only]

Prints ONE JSON line.  The headline (default) is batch-1 decode of the
512-expert, top-10 + shared expert, hidden 4096, intermediate 1024 Q8_0 layer
over 256 distinct hidden states (cycled): a step is one decode token through
the layer (router -> top-K -> K experts -> combine + shared expert), inputs
resident in HBM, no host synchronisation inside the timed region.  The line's
``configs`` object measures the other workloads the same way, each with its
own roofline and CPU baseline:

  c1  64 experts, top-4, hidden 2048, intermediate 512, Q8_0, 1 token
  c3  512 experts, top-3, Q4_K gate/up, Q6_K down, Q8_0 shared expert, decode
  c4  8 consecutive 512-expert top-3 Q2_K/Q3_K layers chained through the
      fused RMSNorm and residual add, forced Zipf(0.456) routing with 37.5 %
      overlap, 512 decode tokens (a step = one token through all 8 layers, in
      one launch; ``per_layer_launches`` times the same chain one launch per
      layer)
  c5  prefill of 512 bf16 tokens through the 512-expert top-10 Q8_0 layer,
      Zipf routing (a step = the whole batch)
  c5r the same batch routed by the layer's fp32 router (router logits and
      top-K of every token inside the timed batch)
  c3p prefill of 512 bf16 tokens through the c3 layer (Q4_K gate/up, Q6_K
      down, Q8_0 shared expert), Zipf routing

``--only`` measures the chosen --config alone (used under the profiler).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import statistics
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer tokens/s at batch 1 and 512; achieved HBM GB/s vs peak"
PEAK_HBM_GBPS = 8000.0
CPU_REPS = 5                 # timed repetitions of the CPU baseline (median reported), after one warm-up
CPU_REP_TARGET_S = 0.6       # wall time one repetition aims at


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_info():
    model, tpc = "", 1
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                model = line.split(":", 1)[1].strip()
            if line.startswith("Thread(s) per core"):
                tpc = int(line.split(":", 1)[1].strip() or 1)
    except (OSError, ValueError):
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    return {"cpu_model": model or platform.processor(), "nproc": os.cpu_count(), "cpus_allowed": allowed,
            "threads_per_core": tpc, "physical_cores_allowed": max(1, allowed // max(tpc, 1)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


# ------------------------------------------------------------------ algorithmic bytes (the rooflines' numerators)

def decode_layer_bytes(cfg) -> int:
    """One decode token through one layer: every expert weight byte touched (K
    routed + shared), the router when it routes, the shared gate vector, x in
    and out."""
    b = cfg.K * cfg.expert_bytes() + cfg.shared_bytes() + 2 * cfg.H * 4
    if cfg.routing == "router":
        b += cfg.E * cfg.H * 4
    if cfg.shared_gate_inp:
        b += cfg.H * 4
    return b


def prefill_bytes(cfg, ids) -> int:
    """One prefill batch: every expert touched once, the shared expert, x (bf16)
    in, out (fp32) out, the router when it routes."""
    uniq = len(np.unique(ids[(ids >= 0) & (ids < cfg.E)]))
    b = uniq * cfg.expert_bytes() + cfg.shared_bytes() + cfg.tokens * cfg.H * (2 + 4)
    if cfg.routing == "router":
        b += cfg.E * cfg.H * 4
    return b


def prefill_gateup_bytes(cfg, ids) -> int:
    """The prefill gate/up phase: gate and up of every expert touched and of
    the shared expert, x rows read once, SwiGLU rows written (fp16 hi + lo)."""
    from winmoe_amd.moe import matrix_bytes
    gt, ut, _ = cfg.types
    uniq = len(np.unique(ids[(ids >= 0) & (ids < cfg.E)]))
    b = uniq * (matrix_bytes(gt, cfg.I, cfg.H) + matrix_bytes(ut, cfg.I, cfg.H))
    b += cfg.tokens * cfg.H * 2 + ids.size * cfg.I * 4
    if cfg.shared_types:
        sgt, sut, _ = cfg.shared_types
        Is = cfg.shared_inter or cfg.I
        b += matrix_bytes(sgt, Is, cfg.H) + matrix_bytes(sut, Is, cfg.H) + cfg.tokens * Is * 4
    return b


def prefill_gateup_kernel(cfg) -> str:
    """What the prefill gate/up phase launches for the workload's formats."""
    from winmoe_amd import TYPE_NAMES
    gt = TYPE_NAMES[cfg.types[0]]
    sgt = TYPE_NAMES[cfg.shared_types[0]] if cfg.shared_types else gt
    what = ("fp16 MFMA over Q8_0 blocks" if gt == "Q8_0" else
            f"fp16 MFMA over {gt} super-blocks, mins from activation sums")
    # pairs per pass: 16 when the batch averages at most 10 (Q8_0) or 4 (K-quant) pairs per
    # expert; then Q2_K .. Q4_K stream two super-blocks per stage when H allows (the library's rules)
    m = 16 if cfg.tokens * cfg.K <= (10 if gt == "Q8_0" else 4) * cfg.E else 32

    def inst_name(t):
        if m == 16 and t in ("Q2_K", "Q3_K", "Q4_K") and cfg.H % 512 == 0:
            return f"k_pf_gemm<1,1,2,{t},16,2>"
        return f"k_pf_gemm<1,1,2,{t},{m},1>" if t in ("Q8_0", "Q6_K") else f"k_pf_gemm<2,1,1,{t},{m},1>"
    inst = {t: inst_name(t) for t in (gt, sgt)}
    if sgt == gt:
        return f"{inst[gt]} (prefill gate+up+SwiGLU: {what}, LDS-DMA ring)"
    return (f"{inst[gt]} + {inst[sgt]} (prefill gate+up+SwiGLU phase: routed {gt} "
            f"launch and shared-expert {sgt} launch; {what})")


def committed_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, calibrated), or None."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def roofline(kernel_desc, kernel, workload, per_launch, launch_us):
    ach = per_launch / (launch_us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBPS, 4), "traffic": committed_traffic(kernel, workload),
            "kernel": kernel_desc, "bytes_per_launch": per_launch, "avg_launch_us": round(launch_us, 2)}


# ------------------------------------------------------------------ workloads on the GPU

class Workload:
    """A synthetic workload resident in HBM and its step function."""

    def __init__(self, name, multi_kernel=False):
        import torch
        from winmoe_amd import synth
        from winmoe_amd.moe import MoELayer
        self.cfg = cfg = synth.CONFIGS[name]
        self.prefill = cfg.x_dtype == "bf16" and cfg.tokens > 1
        self.chained = cfg.n_layers > 1
        self.layers, self.norms = [], []
        g = torch.Generator(device="cuda").manual_seed(2024)
        for i in range(cfg.n_layers):
            sl = synth.build_layer(cfg, layer_index=i, max_tokens=cfg.tokens, multi_kernel=multi_kernel)
            if self.chained:
                # h_{l+1} = h_l + moe_l(rmsnorm(h_l)) (winmoe_inference.c:1659-1668,2041): the norm and the
                # residual add run inside each layer's decode step
                c = sl.cfg
                nw = (1.0 + 0.1 * torch.randn(c.H, generator=g, device="cuda")).float()
                sl.layer = MoELayer(c.H, c.I, sl.layer.E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types,
                                    shared=sl.shared, max_tokens=cfg.tokens, norm_w=nw, add_residual=True)
                self.norms.append(nw)
            self.layers.append(sl)
        self.X = synth.make_hidden(cfg)
        self.routes = None
        if cfg.routing != "router":
            self.routes = []
            for i in range(cfg.n_layers):
                ids, w = synth.forced_routes(cfg, layer_index=i)
                self.routes.append((ids, w, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()))
        # decode outputs [T][H]; a chained stack keeps every layer's stream [L+1][T][H]
        if self.chained:
            self.hs = torch.empty(cfg.n_layers + 1, cfg.tokens, cfg.H, device="cuda")
            self.hs[0] = self.X
            self.stack_out = torch.empty(cfg.tokens, cfg.n_layers, cfg.H, device="cuda")
        # a chained decode runs its layers in one launch per token (wm_moe_decode_stack)
        # unless the per-layer path is asked for
        self.stack = self.chained and not self.prefill and not multi_kernel
        self.outs = torch.empty(cfg.tokens, cfg.H, dtype=torch.float32, device="cuda")
        self._rids = {}

    def step(self, i):
        cfg = self.cfg
        if self.prefill:
            for li, sl in enumerate(self.layers):
                if self.routes is None:
                    sl.layer.prefill(self.X, out=self.outs)
                else:
                    sl.layer.prefill_forced(self.X, self.routes[li][2], self.routes[li][3], out=self.outs)
            return
        t = i % cfg.tokens
        if self.stack:
            from winmoe_amd.moe import decode_stack
            routes = None if self.routes is None else [(r[2][t], r[3][t]) for r in self.routes]
            decode_stack([sl.layer for sl in self.layers], self.X[t], out=self.stack_out[t], routes=routes, step=i)
            return
        for li, sl in enumerate(self.layers):
            if self.chained:
                x, o = self.hs[li, t], self.hs[li + 1, t]
            else:
                x, o = self.X[t], self.outs[t]
            if self.routes is None:
                sl.layer.decode(x, out=o, step=i)
            else:
                sl.layer.decode_forced(x, self.routes[li][2][t], self.routes[li][3][t], out=o, step=i)

    def route_ids(self, li: int = 0):
        """Expert ids [T][K] of layer li: the forced routes, or for a routed
        prefill those the router chose for the batch (read back from the
        prefill workspace after one batch; the inputs are the same every
        batch)."""
        if self.routes is not None:
            return self.routes[li][0]
        if li not in self._rids:
            import torch
            self.step(0)
            torch.cuda.synchronize()
            ids, _ = self.layers[li].layer.prefill_routing(self.cfg.tokens)
            self._rids[li] = ids.cpu().numpy().copy()
        return self._rids[li]

    def status(self):
        return max(sl.layer.prefill_status() if self.prefill else sl.layer.check() for sl in self.layers)

    def tokens_per_step(self):
        return self.cfg.tokens if self.prefill else 1

    def step_bytes(self):
        if self.prefill:
            return prefill_bytes(self.cfg, self.route_ids(0)) * self.cfg.n_layers
        return decode_layer_bytes(self.cfg) * self.cfg.n_layers


def measure(wl, L, steps, warmup, graph):
    """Warm-up, then `steps` steps issued one by one from Python and timed with
    HIP events on the launch stream; with `graph`, the same `steps` steps are
    also captured into one HIP graph and one replay is timed the same way
    (the GPU's own rate, without the host's per-call launch cost); then a
    profiled pass (per-launch events recorded by the library)."""
    import torch
    for i in range(warmup):
        wl.step(i)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    t0 = time.perf_counter()
    for i in range(steps):
        wl.step(warmup + i)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = start.elapsed_time(stop)
    graph_ms = None
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                wl.step(warmup + steps + i)
        g.replay()                                      # warm replay
        torch.cuda.synchronize()
        start.record()
        g.replay()
        stop.record()
        torch.cuda.synchronize()
        graph_ms = start.elapsed_time(stop)
        del g
    n_prof = min(steps, 256)
    L.wm_profile_read(None, None, 0)
    L.wm_profile_enable(1)
    for i in range(n_prof):
        wl.step(warmup + steps + i)
    torch.cuda.synchronize()
    L.wm_profile_enable(0)
    ms_arr = (C.c_double * 8)()
    cnt_arr = (C.c_int64 * 8)()
    L.wm_profile_read(ms_arr, cnt_arr, 8)
    phases = {}
    for p in range(8):
        if cnt_arr[p]:
            phases[L.wm_profile_phase_name(p).decode()] = {"avg_us": round(1000.0 * ms_arr[p] / cnt_arr[p], 3),
                                                           "launches": int(cnt_arr[p])}
    return ev_ms, graph_ms, wall, phases


def entry(wl, L, steps, warmup, multi_kernel=False):
    """Measured record of one workload (without its CPU baseline).  Decode
    steps are timed twice: issued one by one from Python, and as one replay
    of a HIP graph of the steps (the launch cost of one Python call per layer
    per token would otherwise be measured instead of the GPU at the small
    workloads; a replay of a short graph carries a fixed start cost of its
    own); the line reports the faster and names it, the other kept beside."""
    cfg = wl.cfg
    use_graph = not wl.prefill and not multi_kernel
    ev_ms, graph_ms, wall, phases = measure(wl, L, steps, warmup, use_graph)
    eager_ms_per_step = ev_ms / steps
    use_graph_time = graph_ms is not None and graph_ms < ev_ms
    if use_graph_time:
        ev_ms = graph_ms
    ms_per_step = ev_ms / steps
    tokens_per_s = steps * wl.tokens_per_step() / (ev_ms / 1000.0)
    sbytes = wl.step_bytes()
    step_gbps = sbytes / (ms_per_step * 1e-3) / 1e9
    rl = None
    if wl.prefill and "gate_up_swiglu" in phases:
        gu = phases["gate_up_swiglu"]
        rl = roofline(prefill_gateup_kernel(cfg), "k_pf_gemm", cfg.name, prefill_gateup_bytes(cfg, wl.route_ids(0)),
                      gu["avg_us"])
    elif wl.stack:
        # one chained launch per token moves all the layers' bytes
        launch_us = 1000.0 * ev_ms / steps
        rl = roofline("k_decode_stack (the fused decode step of every layer in one launch: one persistent "
                      "workgroup per CU, each layer's output handed to the next in tagged words)",
                      "k_decode_stack", cfg.name, sbytes, launch_us)
    elif not wl.prefill and not multi_kernel:
        # one fused launch per layer per token moves the step's bytes; its
        # average duration is the timed region's event time over the launches
        # in it (back to back on this stream)
        launch_us = 1000.0 * ev_ms / (steps * cfg.n_layers)
        rl = roofline("k_decode_persist (fused decode step: one persistent workgroup per CU, "
                      "1 launch per layer per token)", "k_decode_persist", cfg.name,
                      sbytes // cfg.n_layers, launch_us)
    return {
        "workload": cfg.name, "ms_per_step": round(ms_per_step, 5), "tokens_per_s": round(tokens_per_s, 1),
        "timing": "one replay of a HIP graph of the steps" if use_graph_time else "steps issued from Python",
        "eager_ms_per_step": round(eager_ms_per_step, 5),
        "graph_ms_per_step": round(graph_ms / steps, 5) if graph_ms is not None else None,
        "tokens_per_step": wl.tokens_per_step(), "layers": cfg.n_layers, "steps": steps, "warmup": warmup,
        "roofline": rl, "step_algorithmic_bytes": sbytes, "step_GBps": round(step_gbps, 1),
        "step_hbm_frac": round(step_gbps / PEAK_HBM_GBPS, 4), "wall_s_timed": round(wall, 4),
        "phases_us": phases, "status": wl.status(),
    }


# ------------------------------------------------------------------ CPU baseline

def _host_layer(oracle, sl, experts):
    """The layer in host RAM for the CPU path: router, shared expert and the
    given experts copied from HBM into full-size stacked arrays whose other
    experts are never touched (their pages are never committed)."""
    from winmoe_amd.moe import matrix_bytes
    cfg = sl.cfg
    E, H, I = sl.layer.E, cfg.H, cfg.I
    gt, ut, dt = cfg.types
    per = (matrix_bytes(gt, I, H), matrix_bytes(ut, I, H), matrix_bytes(dt, H, I))
    stacks = [np.zeros(E * p, np.uint8) for p in per]
    for e in experts:
        for arr, src, p in zip(stacks, (sl.gate, sl.up, sl.down), per):
            arr[e * p:(e + 1) * p] = src[e * p:(e + 1) * p].cpu().numpy()
    sh = sl.shared
    return oracle.make_layer(H, I, E, cfg.K, cfg.types,
                             router=None if sl.router is None else sl.router.cpu().numpy(),
                             gate=stacks[0], up=stacks[1], down=stacks[2],
                             shared=None if sh is None else (sh.gate.cpu().numpy(), sh.up.cpu().numpy(),
                                                             sh.down.cpu().numpy()),
                             sh_types=None if sh is None else sh.types,
                             sh_gate_inp=None if (sh is None or sh.gate_inp is None) else sh.gate_inp.cpu().numpy(),
                             I_shared=0 if sh is None else sh.inter)


def cpu_baseline(wl, n_sample):
    """The reference CPU path (oracle/_ref: the reference's own kernels compiled
    from its sources; the oracle port for types the reference has no CPU
    kernel for) on the first n_sample tokens of the workload, on this host.
    One warm-up token, then CPU_REPS timed repetitions over the sample; the
    median repetition gives tokens/s.  Prefill runs the decode path token by
    token, as the reference does for a prompt (winmoe_inference.c:1079,
    2286-2288)."""
    from oracle import oracle
    R = oracle.ref()
    cfg = wl.cfg
    n_sample = min(n_sample, cfg.tokens)
    Xh = wl.X.float().cpu().numpy()
    host = []
    for li, sl in enumerate(wl.layers):
        if wl.routes is not None or wl.prefill:
            experts = np.unique(wl.route_ids(li)[:n_sample])
        else:
            ids, _ = sl.layer.trace()
            experts = np.unique(ids[:n_sample].cpu().numpy())
        host.append(_host_layer(oracle, sl, experts.tolist()))
    norms = [n.cpu().numpy() for n in wl.norms]
    fn = oracle.ref_moe_layer_cpu if R is not None else oracle.moe_layer
    used_port = R is None

    def one_token(t):
        nonlocal used_port
        h = Xh[t]
        for li, L in enumerate(host):
            fi = fw = None
            if wl.routes is not None:
                fi, fw = wl.routes[li][0][t], wl.routes[li][1][t]
            x = h
            if wl.chained:
                x = oracle.ref_rmsnorm(h, norms[li])
            res = fn(L, x, fi, fw)
            if R is not None and res[3] == 1:
                used_port = True
            if wl.chained:
                h = (h + np.asarray(res[2], np.float32)).astype(np.float32)

    t0 = time.perf_counter()
    one_token(0)                                                   # warm-up
    per_tok = max(time.perf_counter() - t0, 1e-4)
    n_rep = int(max(1, min(n_sample, round(CPU_REP_TARGET_S / per_tok))))
    reps = []
    for r in range(CPU_REPS):
        t0 = time.perf_counter()
        for i in range(n_rep):
            one_token((r * n_rep + i) % n_sample)
        reps.append(time.perf_counter() - t0)
    med = statistics.median(reps)
    info = host_info()
    threads = int(os.environ.get("OMP_NUM_THREADS") or info["cpus_allowed"]) if R is not None else 1
    kind = "port" if used_port else "reference"
    what = ("the reference's kernels compiled from its sources" if kind == "reference" else
            "the oracle port (the reference has no CPU kernel for these types)" if R is not None else
            "the oracle port (reference build absent)")
    sample = (f"{n_rep} decode tokens per repetition ({'through all ' + str(cfg.n_layers) + ' layers, ' if wl.chained else ''}"
              f"{n_sample} distinct), 1 warm-up token, median of {CPU_REPS} repetitions "
              f"({', '.join(f'{x:.3f}' for x in reps)} s); weights resident in host RAM; {what}")
    if wl.prefill:
        sample += f"; a prefill batch of {cfg.tokens} tokens is {cfg.tokens} decode tokens (no batched CPU path)"
    return {"value": round(n_rep / med, 2), "unit": "tokens/s", "cores": threads, "kind": kind, "sample": sample,
            "host": info}


# ------------------------------------------------------------------ main

EXTRA = ["c1", "c3", "c4", "c5", "c5r", "c3p"]
CPU_SAMPLE = {"c1": 1, "c2": 16, "c3": 16, "c4": 4, "c5": 8, "c5r": 8, "c3p": 16}


# marks of the persistent step's per-workgroup timeline (include/winmoe_hip.h, wm_workspace_timeline)
TL_MARKS = [(1, "x and router rows in LDS"), (8, "x operand records built"), (2, "own logits stored"),
            (11, "every logit polled"), (3, "routing known")] + \
           [(16 + q, f"SwiGLU of slot position {q} published") for q in range(12)] + \
           [(4, "last SwiGLU published"), (9, "first streaming wave done"), (6, "combine start"), (7, "end")]


def timeline_report(name, steps):
    """The device-clock timeline of the last of `steps` decode steps of the
    workload's first layer (graph replay), per mark the earliest, median and
    latest workgroup, in us from the earliest workgroup start."""
    import numpy as np
    import torch
    from winmoe_amd.moe import MoELayer
    wl = Workload(name)
    if wl.prefill:
        print("--timeline covers the decode workloads (c1-c4)", file=sys.stderr)
        sys.exit(2)
    if wl.stack:
        stack_timeline_report(wl, steps)
        return
    sl, cfg = wl.layers[0], wl.cfg
    c = sl.cfg
    layer = MoELayer(c.H, c.I, sl.layer.E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types, shared=sl.shared,
                     max_tokens=cfg.tokens, timeline=True, norm_w=wl.norms[0] if wl.chained else None,
                     add_residual=wl.chained)
    out = torch.empty(cfg.tokens, cfg.H, device="cuda")

    def step(i):
        t = i % cfg.tokens
        if wl.routes is None:
            layer.decode(wl.X[t], out=out[t], step=i)
        else:
            layer.decode_forced(wl.X[t], wl.routes[0][2][t], wl.routes[0][3][t], out=out[t], step=i)
    for i in range(16):
        step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i)
    g.replay()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    layer.check()
    us = a.elapsed_time(b) * 1000.0 / steps
    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    tl = layer.timeline().cpu().numpy().reshape(-1)[: nwg * 32].reshape(nwg, 32).astype(np.int64)
    tick_us = 1000.0 / wm_clock_khz()
    t0 = tl[:, 0][tl[:, 0] > 0].min()
    print(f"persistent decode step timeline, workload {cfg.name} (layer 0), last of {steps} steps replayed in a HIP "
          f"graph, {nwg} workgroups; us from the earliest workgroup start")
    print(f"{'mark':36s} {'min':>8s} {'median':>8s} {'max':>8s}")
    for k, label in sorted(TL_MARKS, key=lambda m: np.median(tl[:, m[0]][tl[:, m[0]] > 0]) if (tl[:, m[0]] > 0).any()
                           else 1e30):
        v = tl[:, k]
        v = v[v > 0]
        if v.size == 0:
            continue
        r = (v - t0) * tick_us
        print(f"{label:36s} {r.min():8.2f} {np.median(r):8.2f} {r.max():8.2f}")
    print(f"step time over the replay (HIP events): {us:.2f} us")


def stack_timeline_report(wl, steps):
    """The chained launch's timeline: every layer of the last of `steps`
    tokens (graph replay), per layer the median workgroup's marks, in us from
    the earliest workgroup start of the launch."""
    import numpy as np
    import torch
    from winmoe_amd.moe import MoELayer, decode_stack
    cfg = wl.cfg
    layers = []
    for li, sl in enumerate(wl.layers):
        c = sl.cfg
        layers.append(MoELayer(c.H, c.I, sl.layer.E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types,
                               shared=sl.shared, max_tokens=cfg.tokens, timeline=True, norm_w=wl.norms[li],
                               add_residual=True))
    out = torch.empty(cfg.tokens, cfg.n_layers, cfg.H, device="cuda")

    def step(i):
        t = i % cfg.tokens
        routes = None if wl.routes is None else [(r[2][t], r[3][t]) for r in wl.routes]
        decode_stack(layers, wl.X[t], out=out[t], routes=routes, step=i)
    for i in range(16):
        step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i)
    g.replay()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    for m in layers:
        m.check()
    us = a.elapsed_time(b) * 1000.0 / steps
    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    tick_us = 1000.0 / wm_clock_khz()
    tls = [m.timeline().cpu().numpy().reshape(-1)[: nwg * 32].reshape(nwg, 32).astype(np.int64) for m in layers]
    t0 = tls[0][:, 0][tls[0][:, 0] > 0].min()
    marks = [(0, "start"), (8, "x records"), (16, "slot 0 published"), (4, "last SwiGLU"), (6, "combine"),
             (7, "end")]
    print(f"chained decode launch timeline, workload {cfg.name}: {cfg.n_layers} layers in one launch "
          f"(wm_moe_decode_stack), last of {steps} tokens replayed in a HIP graph, {nwg} workgroups; per layer the "
          f"median workgroup's marks, us from the launch's earliest workgroup start")
    print("layer " + " ".join(f"{lab:>17s}" for _, lab in marks) + f" {'latest end':>11s}")
    for li, tl in enumerate(tls):
        row = []
        for k, _ in marks:
            v = tl[:, k]
            v = v[v > 0]
            row.append(f"{np.median((v - t0) * tick_us):17.2f}" if v.size else f"{'-':>17s}")
        print(f"{li:5d} " + " ".join(row) + f" {(tl[:, 7].max() - t0) * tick_us:11.2f}")
    print(f"time per token over the replay (HIP events): {us:.2f} us")


def stream_report(name, n_slots, steps, warmup, layout="packed"):
    """Decode steps of the workload's layer shape with the experts in pinned
    host memory, made resident on demand in a pool of n_slots HBM slots
    (wm_pool_*), Zipf routing with consecutive-token overlap (the forced
    routing of the C4 workload, at this layer's E and K).  layout "packed":
    each expert one slot image in host memory, one copy per miss
    (wm_pool_acquire_packed); "parts": gate, up and down tensors apart, three
    copies per miss (wm_pool_acquire).  One JSON line: tokens/s, misses per
    token, achieved host -> device GB/s."""
    import numpy as np
    import torch
    import winmoe_amd as wm
    from winmoe_amd import synth
    cfg = synth.CONFIGS[name]
    if cfg.x_dtype == "bf16" and cfg.tokens > 1:
        print("--stream-slots covers the decode workloads (c1-c4)", file=sys.stderr)
        sys.exit(2)
    sl = synth.build_layer(cfg, layer_index=0, max_tokens=1)
    c = sl.cfg
    E = sl.layer.E
    parts = [wm.matrix_bytes(c.types[0], c.I, c.H), wm.matrix_bytes(c.types[1], c.I, c.H),
             wm.matrix_bytes(c.types[2], c.H, c.I)]
    log(f"copying {E} experts ({E * sum(parts) / 1e9:.2f} GB) to pinned host memory ({layout})")
    pool = wm.ExpertPool(n_slots, *parts)
    src = []
    if layout == "packed":
        packed = torch.zeros((E, pool.slot_bytes), dtype=torch.uint8, pin_memory=True)
        for o, t, nb in zip(pool.offsets, (sl.gate, sl.up, sl.down), parts):
            packed[:, o:o + nb].copy_(t.view(E, -1)[:, :nb])
    else:
        for t in (sl.gate, sl.up, sl.down):
            h = torch.empty(t.numel(), dtype=torch.uint8, pin_memory=True)
            h.copy_(t)
            src.append(h.view(E, -1))
    layer = pool.layer(c.H, c.I, c.K, c.types, shared=sl.shared, max_tokens=steps + warmup)
    rng = np.random.default_rng(11)
    T = steps + warmup
    ids = synth.zipf_routing(T, E, c.K, rng, overlap=synth.OVERLAP)
    w = torch.from_numpy(synth.softmax_weights(T, c.K, rng)).cuda()
    X = synth.make_hidden(cfg, tokens=min(T, 256))
    out = torch.empty(c.H, device="cuda")
    slots = torch.empty(T, c.K, dtype=torch.int32, device="cuda")

    def step(t):
        if layout == "packed":
            pool.acquire_packed(0, ids[t], packed, out=slots[t])
        else:
            pool.acquire(0, ids[t], *src, out=slots[t])
        layer.decode_forced(X[t % X.shape[0]], slots[t], w[t], out=out, step=t)
        pool.release()
    for t in range(warmup):
        step(t)
    torch.cuda.synchronize()
    h0, m0, b0 = pool.stats()
    t0 = time.perf_counter()
    for t in range(warmup, T):
        step(t)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    layer.check()
    h1, m1, b1 = pool.stats()
    rec = {"report": "host -> HBM expert streaming", "workload": cfg.name, "experts": E, "top_k": c.K,
           "expert_bytes": sum(parts), "host_layout": layout, "pool_slots": n_slots,
           "pool_bytes": n_slots * pool.slot_bytes,
           "routing": f"zipf s={synth.ZIPF_S} overlap={synth.OVERLAP}", "steps": steps, "warmup": warmup,
           "tokens_per_s": round(steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 4),
           "hit_rate": round((h1 - h0) / max(1, (h1 - h0) + (m1 - m0)), 4),
           "misses_per_token": round((m1 - m0) / steps, 3),
           "h2d_GBps": round((b1 - b0) / dt / 1e9, 2), "timing": "host wall clock over the timed steps, "
           "synchronised on both sides; copies on the pool's stream overlap the steps"}
    print(json.dumps(rec))
    pool.close()


def wm_clock_khz():
    import winmoe_amd as wm
    return float(wm.load().wm_device_clock_khz())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "c5r", "c3p"])
    ap.add_argument("--only", action="store_true", help="measure --config alone (no `configs` object)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--multi-kernel", action="store_true",
                    help="run each decode step as per-phase kernel launches instead of the single fused launch")
    ap.add_argument("--timeline", action="store_true",
                    help="print the device-clock timeline of the persistent decode step of --config (its first "
                         "layer) instead of the JSON line")
    ap.add_argument("--stream-slots", type=int, default=0,
                    help="host -> HBM expert streaming: run --config's layer shape with its experts in pinned host "
                         "memory through a pool of this many HBM slots (Zipf routing) and print one report line "
                         "instead of the JSON line")
    ap.add_argument("--stream-layout", default="packed", choices=["packed", "parts"],
                    help="with --stream-slots: host copies of the experts as one slot image each (one copy per miss) "
                         "or as separate gate / up / down tensors (three copies per miss)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run 4 plain device copies and 4 read-only reductions of this many MiB (kernels of "
                         "known traffic for the rocprofv3 FETCH_SIZE / WRITE_SIZE calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    import winmoe_amd as wm

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    L = wm.load()

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 18              # floats
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        acc = torch.zeros((), device="cuda")
        for _ in range(4):
            acc += src.sum()                             # reads n floats, writes a few bytes
        torch.cuda.synchronize()
        del src, dst, acc
        log(f"ran 4 device copies and 4 reductions of {args.copy_calibration_mib} MiB")

    def run(name, steps, warmup, headline):
        log(f"building {name} on {torch.cuda.get_device_name(0)}")
        t_build = time.perf_counter()
        wl = Workload(name, multi_kernel=args.multi_kernel and headline)
        torch.cuda.synchronize()
        log(f"built in {time.perf_counter() - t_build:.1f} s")
        e = entry(wl, L, steps, warmup, multi_kernel=args.multi_kernel and headline)
        if wl.stack:
            # the same chain one launch per layer (the drop-in per-layer calls)
            wl.stack = False
            e2 = entry(wl, L, steps, warmup)
            wl.stack = True
            e["per_layer_launches"] = {k: e2[k] for k in ("ms_per_step", "tokens_per_s", "timing", "roofline")}
        if not args.no_cpu_baseline:
            log(f"timing the reference CPU path on this host ({name})")
            e["cpu_baseline"] = cpu_baseline(wl, CPU_SAMPLE[name])
        else:
            e["cpu_baseline"] = None
        cfg = wl.cfg
        e["config"] = {"workload": cfg.name, "experts": cfg.E, "top_k": cfg.K, "hidden": cfg.H, "inter": cfg.I,
                       "types": [wm.TYPE_NAMES[t] for t in cfg.types],
                       "shared_types": [wm.TYPE_NAMES[t] for t in cfg.shared_types] if cfg.shared_types else None,
                       "layers": cfg.n_layers, "routing": cfg.routing,
                       "batch": cfg.tokens if wl.prefill else 1, "distinct_tokens": cfg.tokens,
                       "path": "prefill" if wl.prefill else ("multi-kernel" if args.multi_kernel and headline
                                                             else "fused, the layers chained in one launch"
                                                             if wl.stack else "fused")}
        e["dtype"] = ("fp16 MFMA (quantised weights exact in fp16, x fp16 per-token scaled, SwiGLU output fp16 hi+lo) "
                      "-> fp32" if wl.prefill else
                      "int8 dot (quantised weights x int8 activation digits) -> int32, fp32 scales/accumulation")
        del wl
        torch.cuda.empty_cache()
        return e

    if args.timeline:
        timeline_report(args.config, min(args.steps, 256))
        return
    if args.stream_slots > 0:
        stream_report(args.config, args.stream_slots, min(args.steps, 256), min(args.warmup, 64), args.stream_layout)
        return

    head = run(args.config, args.steps, args.warmup, True)
    configs = None
    if not args.only:
        configs = {}
        for name in EXTRA:
            if name == args.config:
                continue
            configs[name] = run(name, args.steps, args.warmup, False)
    result = {
        "metric": METRIC, "value": head["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": head["dtype"],
        "data": "synthetic (seeded N(0,0.02) weights quantised on device, N(0,1) hidden states)",
        "config": head["config"], "roofline": head["roofline"], "cpu_baseline": head["cpu_baseline"],
        "timing": head["timing"], "eager_ms_per_step": head["eager_ms_per_step"],
        "graph_ms_per_step": head["graph_ms_per_step"],
        "step_algorithmic_bytes": head["step_algorithmic_bytes"], "step_GBps": head["step_GBps"],
        "step_hbm_frac": head["step_hbm_frac"], "wall_s_timed": head["wall_s_timed"],
        "phases_us": head["phases_us"], "status": head["status"],
        "configs": configs,
    }
    if "per_layer_launches" in head:
        result["per_layer_launches"] = head["per_layer_launches"]
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
