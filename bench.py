"""Benchmark of the MoE expert-layer hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2] [--gpus 1] [--no-cpu-baseline]

A step is one decode token through the layer (router -> top-K -> K experts ->
combine + shared expert), inputs resident in HBM, no host synchronisation
inside the timed region.  Prints ONE JSON line.  Default workload: 512
experts, top-10 + shared expert, hidden 4096, intermediate 1024, Q8_0, batch-1
decode over 256 distinct hidden states (cycled).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer tokens/s at batch 1 and 512; achieved HBM GB/s vs peak"
PEAK_HBM_GBPS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_info():
    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                model = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return {"cpu_model": model or platform.processor(), "nproc": os.cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def step_bytes(cfg) -> int:
    """Algorithmic bytes of one decode step: every expert weight byte touched
    (K routed + shared), router, shared gate vector, activation in/out."""
    b = cfg.K * cfg.expert_bytes() + cfg.shared_bytes() + 2 * cfg.H * 4
    if cfg.routing == "router":
        b += cfg.E * cfg.H * 4
    if cfg.shared_gate_inp:
        b += cfg.H * 4
    return b * cfg.n_layers


def prefill_bytes(cfg, ids) -> int:
    """Algorithmic bytes of one prefill batch: every expert touched once,
    the shared expert, x (bf16) in, out (fp32) out, the router when it routes."""
    uniq = len(np.unique(ids[(ids >= 0) & (ids < cfg.E)]))
    b = uniq * cfg.expert_bytes() + cfg.shared_bytes() + cfg.tokens * cfg.H * (2 + 4)
    if cfg.routing == "router":
        b += cfg.E * cfg.H * 4
    return b


def prefill_gateup_bytes(cfg, ids) -> int:
    """Algorithmic bytes of the prefill gate/up launch: gate and up of every
    expert touched (and the shared one), x rows read once, SwiGLU rows written."""
    from winmoe_amd.moe import matrix_bytes
    gt, ut, _ = cfg.types
    uniq = len(np.unique(ids[(ids >= 0) & (ids < cfg.E)]))
    b = uniq * (matrix_bytes(gt, cfg.I, cfg.H) + matrix_bytes(ut, cfg.I, cfg.H))
    b += cfg.tokens * cfg.H * 2 + ids.size * cfg.I * 4
    return b


def gateup_bytes(cfg) -> int:
    """Algorithmic bytes of one launch of the gate/up + SwiGLU kernel (weights + act out)."""
    from winmoe_amd.moe import matrix_bytes
    gt, ut, _ = cfg.types
    per = matrix_bytes(gt, cfg.I, cfg.H) + matrix_bytes(ut, cfg.I, cfg.H) + cfg.I * 4
    n = cfg.K
    if cfg.shared_types and tuple(cfg.shared_types) == tuple(cfg.types) and (cfg.shared_inter or cfg.I) == cfg.I:
        n += 1
    return n * per


def measured_traffic(cfg):
    """HBM bytes per launch of the fused kernel from the committed rocprofv3
    PMC summary for this workload (FETCH_SIZE + WRITE_SIZE, scaled by the copy
    kernel calibration), or None when there is none."""
    path = os.path.join(ROOT, "profiles", f"k_decode_persist_{cfg.name}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(layers, X, routes, budget_s: float):
    """Reference CPU path (oracle/_ref, compiled from the reference sources) on
    the same layer, weights copied to host RAM; falls back to the oracle port."""
    from oracle import oracle
    R = oracle.ref()
    kind = "reference" if R is not None else "port"
    host_layers = []
    for sl in layers:
        cfg = sl.cfg
        sh = sl.shared
        L = oracle.make_layer(cfg.H, cfg.I, sl.layer.E, cfg.K, cfg.types,
                              router=None if sl.router is None else sl.router.cpu().numpy(),
                              gate=sl.gate.cpu().numpy(), up=sl.up.cpu().numpy(), down=sl.down.cpu().numpy(),
                              shared=None if sh is None else (sh.gate.cpu().numpy(), sh.up.cpu().numpy(),
                                                              sh.down.cpu().numpy()),
                              sh_types=None if sh is None else sh.types,
                              sh_gate_inp=None if (sh is None or sh.gate_inp is None) else sh.gate_inp.cpu().numpy(),
                              I_shared=0 if sh is None else sh.inter)
        host_layers.append(L)
    Xh = X.float().cpu().numpy()
    fn = oracle.ref_moe_layer_cpu if R is not None else oracle.moe_layer
    n = 0
    used_port = False
    t0 = time.perf_counter()
    while True:
        t = n % Xh.shape[0]
        for li, L in enumerate(host_layers):
            fi = fw = None
            if routes is not None:
                fi, fw = routes[li][0][t], routes[li][1][t]
            res = fn(L, Xh[t], fi, fw)
            if R is not None and res[3] == 1:
                used_port = True
        n += 1
        el = time.perf_counter() - t0
        if (el >= budget_s and n >= 2) or n >= 4096:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1) if R is not None else 1
    if used_port:
        kind = "port"
    return {"value": n / el, "unit": "tokens/s", "cores": threads, "kind": kind,
            "sample": f"{n} decode tokens of the same layer(s) ({el:.1f} s), weights resident in host RAM, "
                      f"{'reference kernels compiled from the reference sources' if kind == 'reference' else 'oracle port'}",
            "host": host_info()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--multi-kernel", action="store_true",
                    help="run each step as per-phase kernel launches instead of the single fused launch")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run 4 plain device copies of this many MiB (reference kernel of known traffic "
                         "for rocprofv3 FETCH_SIZE / WRITE_SIZE calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    import winmoe_amd as wm
    from winmoe_amd import synth

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    L = wm.load()
    cfg = synth.CONFIGS[args.config]
    log(f"building {cfg.name} on {torch.cuda.get_device_name(0)}")
    t_build = time.perf_counter()
    layers = [synth.build_layer(cfg, layer_index=i, max_tokens=cfg.tokens, multi_kernel=args.multi_kernel)
              for i in range(cfg.n_layers)]
    X = synth.make_hidden(cfg)
    routes = None
    if cfg.routing != "router":
        routes = []
        for i in range(cfg.n_layers):
            ids, w = synth.forced_routes(cfg, layer_index=i)
            routes.append((ids, w, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()))
    outs = torch.empty(cfg.tokens, cfg.H, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    log(f"built in {time.perf_counter() - t_build:.1f} s")

    prefill = cfg.x_dtype == "bf16" and cfg.tokens > 1     # one step = the whole batch through the layer

    def step(i):
        if prefill:
            for li, sl in enumerate(layers):
                if routes is None:
                    sl.layer.prefill(X, out=outs)
                else:
                    sl.layer.prefill_forced(X, routes[li][2], routes[li][3], out=outs)
            return
        t = i % cfg.tokens
        x = X[t]
        for li, sl in enumerate(layers):
            o = outs[t]
            if routes is None:
                sl.layer.decode(x, out=o, step=i)
            else:
                sl.layer.decode_forced(x, routes[li][2][t], routes[li][3][t], out=o, step=i)

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 18              # floats
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"ran 4 device copies of {args.copy_calibration_mib} MiB")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K steps back to back, inputs resident, no profiling
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = start.elapsed_time(stop)

    # ---- roofline pass: per-launch duration of the dominant kernel from HIP
    # events recorded by the library around each launch, on its stream
    n_prof = min(args.steps, 256)
    L.wm_profile_read(None, None, 0)
    L.wm_profile_enable(1)
    for i in range(n_prof):
        step(args.warmup + args.steps + i)
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
    st = max(sl.layer.prefill_status() if prefill else sl.layer.status() for sl in layers)
    ms_per_step = ev_ms / args.steps
    tokens_per_s = args.steps * (cfg.tokens if prefill else 1) / (ev_ms / 1000.0)
    sbytes = prefill_bytes(cfg, routes[0][0]) * cfg.n_layers if prefill else step_bytes(cfg)
    step_gbps = sbytes / (ms_per_step * 1e-3) / 1e9
    roofline = None
    if prefill and "gate_up_swiglu" in phases:
        gu = phases["gate_up_swiglu"]
        per_launch = prefill_gateup_bytes(cfg, routes[0][0])
        ach = per_launch / (gu["avg_us"] * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                    "frac": round(ach / PEAK_HBM_GBPS, 4), "traffic": None,
                    "kernel": "k_pf_gemm<2,1,1> (prefill gate+up+SwiGLU: fp16 MFMA over Q8_0 blocks, LDS-DMA ring)",
                    "bytes_per_launch": per_launch, "avg_launch_us": round(gu["avg_us"], 2)}
    elif prefill:
        pass
    elif not args.multi_kernel:
        # one fused launch per layer per token moves the whole step's bytes;
        # its average duration is the timed region's event time over the
        # launches in it (they run back to back on this stream)
        launch_us = 1000.0 * ev_ms / (args.steps * cfg.n_layers)
        per_launch = sbytes // cfg.n_layers
        ach = per_launch / (launch_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                    "frac": round(ach / PEAK_HBM_GBPS, 4), "traffic": measured_traffic(cfg),
                    "kernel": "k_decode_persist (fused decode step: one persistent workgroup per CU, "
                              "1 launch per layer per token)",
                    "bytes_per_launch": per_launch, "avg_launch_us": round(launch_us, 2)}
    elif "gate_up_swiglu" in phases:
        gu = phases["gate_up_swiglu"]
        per_launch = gateup_bytes(cfg)
        ach = per_launch / (gu["avg_us"] * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                    "frac": round(ach / PEAK_HBM_GBPS, 4), "traffic": None,
                    "kernel": "k_gateup (gate+up+SwiGLU)", "bytes_per_launch": per_launch,
                    "avg_launch_us": round(gu["avg_us"], 2)}
    result = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("fp16 MFMA (int8 weights exact in fp16, x fp16 per-token scaled, SwiGLU output fp16 hi+lo) -> fp32"
                  if prefill else "int8 dot (quantised weights x int8 activation digits) -> int32, fp32 scales/accumulation"),
        "data": "synthetic (seeded N(0,0.02) weights quantised on device, N(0,1) hidden states)",
        "config": {"workload": cfg.name, "experts": cfg.E, "top_k": cfg.K, "hidden": cfg.H, "inter": cfg.I,
                   "types": [wm.TYPE_NAMES[t] for t in cfg.types],
                   "shared_types": [wm.TYPE_NAMES[t] for t in cfg.shared_types] if cfg.shared_types else None,
                   "layers": cfg.n_layers, "routing": cfg.routing, "batch": cfg.tokens if prefill else 1,
                   "distinct_tokens": cfg.tokens,
                   "path": "prefill" if prefill else ("multi-kernel" if args.multi_kernel else "fused")},
        "roofline": roofline,
        "step_algorithmic_bytes": sbytes, "step_GBps": round(step_gbps, 1),
        "step_hbm_frac": round(step_gbps / PEAK_HBM_GBPS, 4),
        "wall_s_timed": round(wall, 4), "phases_us": phases, "status": st,
    }
    if not args.no_cpu_baseline:
        log("timing the reference CPU path on this host")
        result["cpu_baseline"] = cpu_baseline(layers, X, routes, args.cpu_budget)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
