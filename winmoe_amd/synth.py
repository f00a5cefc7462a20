"""Seeded synthetic MoE layers and routing traces for the benchmark configurations.

Weights are drawn on the device from N(0, 0.02) (torch's generator on the
layer's device) and quantised with the library's own block quantisers; router
weights are fp32 N(0, 0.02); hidden states N(0, 1).  Forced routing follows a
Zipf popularity p_r ~ r^-s over a per-layer random permutation of expert ids
(work/sim/moe_cache_simulator.py:306-324), optionally with a consecutive-token
overlap (work/traces/processed/olmoe_trace_stats.json: s = 0.4561, overlap
0.3748).  Routing weights of forced routes are softmax(N(0, 1)) over the K ids.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import Q2_K, Q3_K, Q4_K, Q6_K, Q8_0
from .moe import MoELayer, SharedExpert, matrix_bytes, quantize_into

ZIPF_S = 0.456
OVERLAP = 0.375


@dataclass(frozen=True)
class LayerConfig:
    name: str
    E: int
    K: int
    H: int
    I: int
    types: Tuple[int, int, int]
    shared_types: Optional[Tuple[int, int, int]] = None
    shared_inter: int = 0
    shared_gate_inp: bool = False
    tokens: int = 1
    routing: str = "router"          # "router" | "zipf" | "zipf_overlap"
    n_layers: int = 1
    x_dtype: str = "f32"             # "f32" | "bf16"
    seed: int = 0

    def expert_bytes(self) -> int:
        gt, ut, dt = self.types
        return (matrix_bytes(gt, self.I, self.H) + matrix_bytes(ut, self.I, self.H) +
                matrix_bytes(dt, self.H, self.I))

    def shared_bytes(self) -> int:
        if not self.shared_types:
            return 0
        Is = self.shared_inter or self.I
        gt, ut, dt = self.shared_types
        return matrix_bytes(gt, Is, self.H) + matrix_bytes(ut, Is, self.H) + matrix_bytes(dt, self.H, Is)


CONFIGS = {
    "c1": LayerConfig("e64_k4_h2048_i512_q8_0", E=64, K=4, H=2048, I=512, types=(Q8_0, Q8_0, Q8_0), tokens=1),
    "c2": LayerConfig("e512_k10_h4096_i1024_q8_0_shared_decode", E=512, K=10, H=4096, I=1024,
                      types=(Q8_0, Q8_0, Q8_0), shared_types=(Q8_0, Q8_0, Q8_0), shared_inter=1024,
                      shared_gate_inp=True, tokens=256),
    "c3": LayerConfig("e512_k3_h4096_i1024_q4k_q6k_shared_q8_0_decode", E=512, K=3, H=4096, I=1024,
                      types=(Q4_K, Q4_K, Q6_K), shared_types=(Q8_0, Q8_0, Q8_0), shared_inter=1024,
                      shared_gate_inp=True, tokens=256),
    "c4": LayerConfig("8x_e512_k3_h4096_i1024_q2k_q3k_zipf_decode", E=512, K=3, H=4096, I=1024,
                      types=(Q2_K, Q2_K, Q3_K), tokens=512, routing="zipf_overlap", n_layers=8),
    "c5": LayerConfig("e512_k10_h4096_i1024_q8_0_prefill512_zipf", E=512, K=10, H=4096, I=1024,
                      types=(Q8_0, Q8_0, Q8_0), tokens=512, routing="zipf", x_dtype="bf16"),
    # the c5 layer routed by its own router (fp32 N(0, 0.02) weights: close to
    # uniform routing, every expert used), so the batch includes the router
    # logits and top-K of all 512 tokens
    "c5r": LayerConfig("e512_k10_h4096_i1024_q8_0_prefill512_router", E=512, K=10, H=4096, I=1024,
                       types=(Q8_0, Q8_0, Q8_0), tokens=512, routing="router", x_dtype="bf16"),
    # the c3 layer (K-quant experts, Q8_0 shared expert) under a 512-token prefill
    "c3p": LayerConfig("e512_k3_h4096_i1024_q4k_q6k_shared_q8_0_prefill512_zipf", E=512, K=3, H=4096, I=1024,
                       types=(Q4_K, Q4_K, Q6_K), shared_types=(Q8_0, Q8_0, Q8_0), shared_inter=1024,
                       shared_gate_inp=True, tokens=512, routing="zipf", x_dtype="bf16"),
}


def _fill_quantised(out: torch.Tensor, qtype: int, n_mats: int, rows: int, cols: int, g: torch.Generator,
                    chunk_weights: int = 1 << 26) -> None:
    per = matrix_bytes(qtype, rows, cols)
    n_w = rows * cols
    mats_per_chunk = max(1, chunk_weights // n_w)
    for m0 in range(0, n_mats, mats_per_chunk):
        m1 = min(n_mats, m0 + mats_per_chunk)
        x = torch.randn((m1 - m0) * n_w, generator=g, device=out.device, dtype=torch.float32)
        x.mul_(0.02)
        quantize_into(x, qtype, out[m0 * per:m1 * per])
        del x


@dataclass
class SynthLayer:
    cfg: LayerConfig
    layer: MoELayer
    router: Optional[torch.Tensor]
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor
    shared: Optional[SharedExpert] = None
    extra: dict = field(default_factory=dict)


def build_layer(cfg: LayerConfig, device="cuda", layer_index: int = 0, max_tokens: Optional[int] = None,
                E: Optional[int] = None, multi_kernel: bool = False) -> SynthLayer:
    """Generate one layer of cfg on device.  E may shrink the expert count for tests."""
    E = E or cfg.E
    g = torch.Generator(device=device)
    g.manual_seed(1_000_003 * cfg.seed + 7919 * layer_index + 1)
    gt, ut, dt = cfg.types
    gate = torch.empty(E * matrix_bytes(gt, cfg.I, cfg.H), dtype=torch.uint8, device=device)
    up = torch.empty(E * matrix_bytes(ut, cfg.I, cfg.H), dtype=torch.uint8, device=device)
    down = torch.empty(E * matrix_bytes(dt, cfg.H, cfg.I), dtype=torch.uint8, device=device)
    _fill_quantised(gate, gt, E, cfg.I, cfg.H, g)
    _fill_quantised(up, ut, E, cfg.I, cfg.H, g)
    _fill_quantised(down, dt, E, cfg.H, cfg.I, g)
    router = None
    if cfg.routing == "router":
        router = torch.randn(E, cfg.H, generator=g, device=device, dtype=torch.float32).mul_(0.02)
    shared = None
    if cfg.shared_types:
        Is = cfg.shared_inter or cfg.I
        sgt, sut, sdt = cfg.shared_types
        sg = torch.empty(matrix_bytes(sgt, Is, cfg.H), dtype=torch.uint8, device=device)
        su = torch.empty(matrix_bytes(sut, Is, cfg.H), dtype=torch.uint8, device=device)
        sd = torch.empty(matrix_bytes(sdt, cfg.H, Is), dtype=torch.uint8, device=device)
        _fill_quantised(sg, sgt, 1, Is, cfg.H, g)
        _fill_quantised(su, sut, 1, Is, cfg.H, g)
        _fill_quantised(sd, sdt, 1, cfg.H, Is, g)
        gi = None
        if cfg.shared_gate_inp:
            gi = torch.randn(cfg.H, generator=g, device=device, dtype=torch.float32).mul_(0.02)
        shared = SharedExpert(sg, su, sd, tuple(cfg.shared_types), gi, Is)
    layer = MoELayer(cfg.H, cfg.I, E, cfg.K, router, gate, up, down, cfg.types, shared=shared,
                     max_tokens=max_tokens or max(cfg.tokens, 1), multi_kernel=multi_kernel)
    return SynthLayer(cfg, layer, router, gate, up, down, shared)


def twin_layer(sl: SynthLayer, multi_kernel: bool, flags: int = 0) -> MoELayer:
    """A second MoELayer over the same device tensors (own workspace); flags
    are extra wm_layer_desc.flags bits (the kernel choice)."""
    c = sl.cfg
    m = MoELayer(c.H, c.I, sl.layer.E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types, shared=sl.shared,
                 max_tokens=sl.layer.max_tokens, multi_kernel=multi_kernel)
    m.desc.flags |= flags
    return m


def make_hidden(cfg: LayerConfig, device="cuda", tokens: Optional[int] = None, seed_offset: int = 0) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(1_000_003 * cfg.seed + 424242 + seed_offset)
    T = tokens or cfg.tokens
    x = torch.randn(T, cfg.H, generator=g, device=device, dtype=torch.float32)
    return x.to(torch.bfloat16) if cfg.x_dtype == "bf16" else x


# ------------------------------------------------------------------ forced routing

def zipf_probs(E: int, s: float = ZIPF_S) -> np.ndarray:
    r = np.arange(1, E + 1, dtype=np.float64)
    w = 1.0 / r ** s
    return w / w.sum()


def zipf_routing(T: int, E: int, K: int, rng: np.random.Generator, s: float = ZIPF_S,
                 overlap: float = 0.0) -> np.ndarray:
    """[T][K] expert ids: Zipf popularity over a random id permutation; with
    overlap > 0, each slot keeps an id of the previous token's set with that
    probability (no duplicates within a token)."""
    perm = rng.permutation(E)
    p = zipf_probs(E, s)
    ids = np.zeros((T, K), dtype=np.int32)
    prev: List[int] = []
    for t in range(T):
        chosen: List[int] = []
        for k in range(K):
            keep = [e for e in prev if e not in chosen]
            if overlap > 0 and keep and rng.random() < overlap:
                chosen.append(int(keep[rng.integers(len(keep))]))
                continue
            mask = np.ones(E, bool)
            if chosen:
                inv = np.argsort(perm)
                mask[inv[np.array(chosen)]] = False
            q = p * mask
            q /= q.sum()
            r = int(rng.choice(E, p=q))
            chosen.append(int(perm[r]))
        ids[t] = chosen
        prev = chosen
    return ids


def softmax_weights(T: int, K: int, rng: np.random.Generator) -> np.ndarray:
    s = rng.standard_normal((T, K))
    e = np.exp(s - s.max(axis=1, keepdims=True))
    return (e / e.sum(axis=1, keepdims=True)).astype(np.float32)


def routing_stats(ids: np.ndarray, E: int) -> dict:
    """Generator self-checks: Zipf slope of the top-30 log-frequency
    (capture_olmoe_traces.py:192-196) and mean consecutive overlap (:218-224)."""
    T, K = ids.shape
    freq = np.bincount(ids.reshape(-1), minlength=E)
    f = np.sort(freq)[::-1]
    f = f[f > 0][:30].astype(np.float64)
    slope = -np.polyfit(np.log(np.arange(1, len(f) + 1)), np.log(f), 1)[0] if len(f) >= 3 else 0.0
    ovl = [len(set(ids[t - 1]) & set(ids[t])) / K for t in range(1, T)]
    return {"zipf_slope_top30": float(slope), "mean_overlap": float(np.mean(ovl)) if ovl else 0.0,
            "max_count": int(freq.max()), "min_count": int(freq.min()), "experts_touched": int((freq > 0).sum())}


def forced_routes(cfg: LayerConfig, layer_index: int = 0, E: Optional[int] = None, tokens: Optional[int] = None):
    """(ids int32 [T][K], w fp32 [T][K]) numpy arrays for a forced-routing config."""
    E = E or cfg.E
    T = tokens or cfg.tokens
    rng = np.random.default_rng([cfg.seed, 17, layer_index])
    ov = OVERLAP if cfg.routing == "zipf_overlap" else 0.0
    ids = zipf_routing(T, E, cfg.K, rng, overlap=ov)
    w = softmax_weights(T, cfg.K, rng)
    return ids, w
