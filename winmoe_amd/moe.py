"""PyTorch-ROCm host API of the MoE expert-layer path.

Mirrors the reference's entry points on device tensors:

* ``router_topk``      engine/runtime/transformer.h:107-152 (+ verify_router.py:71-84)
* ``quant_matvec``     engine/runtime/transformer.h:157-194
* ``dequantize`` / ``dequant_q8_0_row`` / ``dequant_q4k_block``
                       q8_dequant.h:116-126, validate_l0.py:32-45, verify_expert.py:55-88 (ggml order)
* ``expert_ffn``       expert_ffn.h:48-74, gpu_expert_ffn_fused (gpu_offload.cu:718-751)
* ``MoELayer.decode``  the MoE block of winmoe_inference.c:1684-2027 for one token
* ``MoELayer.prefill`` the same block for a batch of prompt tokens

Torch is used only for device memory and streams; every computation runs in
libwinmoe_hip.so.  Tensors must live on the current HIP device.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import BLOCK_BYTES, BLOCK_ELEMS, LayerDesc, check, load


def _stream(stream=None) -> C.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _p(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, dtype, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def matrix_bytes(qtype: int, rows: int, cols: int) -> int:
    return rows * (cols // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]


def _ws(nbytes: int, device) -> torch.Tensor:
    # 256-byte aligned (the caching allocator hands out >= 512-byte aligned blocks)
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# ------------------------------------------------------------------ block ops

def dequantize(blocks: torch.Tensor, qtype: int, stream=None) -> torch.Tensor:
    """fp32 weights of raw blocks (uint8, whole blocks).  Bit-exact with the oracle."""
    _need(blocks, torch.uint8, "blocks")
    bs = BLOCK_BYTES[qtype]
    if blocks.numel() % bs:
        raise ValueError("blocks must hold whole blocks")
    nb = blocks.numel() // bs
    out = torch.empty(nb * BLOCK_ELEMS[qtype], dtype=torch.float32, device=blocks.device)
    check(load().wm_dequant(qtype, _p(blocks), nb, _p(out), _stream(stream)), "wm_dequant")
    return out


def dequant_q8_0_row(data: torch.Tensor, offset: int, n_elements: int) -> torch.Tensor:
    """validate_l0.py:32-45 on device: one Q8_0 row of n_elements starting at byte offset."""
    nb = n_elements // 32
    return dequantize(data[offset:offset + nb * 34], _lib.Q8_0)


def dequant_q4k_block(data: torch.Tensor, offset: int) -> torch.Tensor:
    """One Q4_K block in the ggml order (q4k_dequant.h:129-155), not verify_expert.py's order."""
    return dequantize(data[offset:offset + 144], _lib.Q4_K)


def quantize(x: torch.Tensor, qtype: int, stream=None) -> torch.Tensor:
    """Quantise fp32 values (length a multiple of the block size) into raw blocks."""
    _need(x, torch.float32, "x")
    n = x.numel()
    if n % BLOCK_ELEMS[qtype]:
        raise ValueError("length must be a multiple of the block size")
    out = torch.empty(n // BLOCK_ELEMS[qtype] * BLOCK_BYTES[qtype], dtype=torch.uint8, device=x.device)
    check(load().wm_quantize(qtype, _p(x), n, _p(out), _stream(stream)), "wm_quantize")
    return out


def quantize_into(x: torch.Tensor, qtype: int, out: torch.Tensor, stream=None) -> None:
    _need(x, torch.float32, "x")
    n = x.numel()
    if out.numel() != n // BLOCK_ELEMS[qtype] * BLOCK_BYTES[qtype]:
        raise ValueError("output size mismatch")
    check(load().wm_quantize(qtype, _p(x), n, _p(out), _stream(stream)), "wm_quantize")


def quant_matvec(W: torch.Tensor, x: torch.Tensor, out_dim: int, in_dim: int, qtype: int,
                 stream=None) -> torch.Tensor:
    """y = W x for one raw quantised matrix [out_dim][in_dim/QK] (transformer.h:157-194)."""
    _need(W, torch.uint8, "W")
    _need(x, torch.float32, "x")
    if W.numel() < matrix_bytes(qtype, out_dim, in_dim) or x.numel() != in_dim:
        raise ValueError("shape mismatch")
    y = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    ws = _ws((in_dim // 64) * 160, x.device)
    check(load().wm_quant_matvec(qtype, _p(W), _p(x), out_dim, in_dim, _p(y), _p(ws), ws.numel(),
                                 _stream(stream)), "wm_quant_matvec")
    return y


def q8_0_matvec(W: torch.Tensor, x: torch.Tensor, out_dim: int, in_dim: int) -> torch.Tensor:
    """verify_3layers.py:85-101 on device."""
    return quant_matvec(W, x, out_dim, in_dim, _lib.Q8_0)


def router_logits(hidden: torch.Tensor, gate_weights: torch.Tensor, stream=None) -> torch.Tensor:
    """fp32 router logits [E] in the reference's accumulation order (gpu_router on device)."""
    _need(hidden, torch.float32, "hidden")
    _need(gate_weights, torch.float32, "gate_weights")
    E, H = gate_weights.shape
    out = torch.empty(E, dtype=torch.float32, device=hidden.device)
    check(load().wm_router_logits(_p(hidden), _p(gate_weights), H, E, _p(out), _stream(stream)), "wm_router_logits")
    return out


def router_topk(hidden: torch.Tensor, gate_weights: torch.Tensor, K: int, stream=None):
    """Reference-order fp32 router logits, top-K ids (desc logit, ties to the lower
    index) and softmax weights over the K picks.  gate_weights is [E][H] fp32."""
    _need(hidden, torch.float32, "hidden")
    _need(gate_weights, torch.float32, "gate_weights")
    E, H = gate_weights.shape
    if hidden.numel() != H:
        raise ValueError("hidden size mismatch")
    L = load()
    ids = torch.empty(K, dtype=torch.int32, device=hidden.device)
    w = torch.empty(K, dtype=torch.float32, device=hidden.device)
    ws = _ws(L.wm_router_workspace_size(E), hidden.device)
    check(L.wm_router_topk(_p(hidden), _p(gate_weights), H, E, K, _p(ids), _p(w), _p(ws), ws.numel(),
                           _stream(stream)), "wm_router_topk")
    return ids, w


def expert_ffn(gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, x: torch.Tensor, H: int, I: int,
               types: Sequence[int], stream=None) -> torch.Tensor:
    """down(SwiGLU(gate x, up x)) for one expert's raw blocks (any supported types)."""
    for t, n in ((gate, "gate"), (up, "up"), (down, "down")):
        _need(t, torch.uint8, n)
    _need(x, torch.float32, "x")
    L = load()
    out = torch.empty(H, dtype=torch.float32, device=x.device)
    ws = _ws(L.wm_expert_workspace_size(H, I), x.device)
    gt, ut, dt = types
    check(L.wm_expert_ffn(_p(gate), gt, _p(up), ut, _p(down), dt, _p(x), H, I, _p(out), _p(ws), ws.numel(),
                          _stream(stream)), "wm_expert_ffn")
    return out


# ------------------------------------------------------------------ layer

@dataclass
class SharedExpert:
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor
    types: tuple
    gate_inp: Optional[torch.Tensor] = None   # fp32 [H] sigmoid gate, or None
    inter: int = 0                            # 0 = routed intermediate


class MoELayer:
    """One MoE layer over raw GGUF expert tensors resident in HBM.

    gate_exps / up_exps: uint8, stacked [E][I rows][H/QK blocks]; down_exps:
    [E][H rows][I/QK blocks] -- the per-expert slicing of the reference
    (winmoe_inference.c:467-489).  ``strides`` overrides the per-expert byte
    stride (e.g. a GGUF tensor's data_size / E).  The workspace (routing trace
    of ``max_tokens`` entries, hit counters, scratch) is allocated once.
    A decode step is one fused kernel launch; ``multi_kernel=True`` runs the
    same step as per-phase launches (bit-identical, used as a cross-check).
    """

    def __init__(self, H: int, I: int, E: int, K: int, router: Optional[torch.Tensor], gate_exps: torch.Tensor,
                 up_exps: torch.Tensor, down_exps: torch.Tensor, types: Sequence[int],
                 shared: Optional[SharedExpert] = None, max_tokens: int = 256, strides=(0, 0, 0),
                 multi_kernel: bool = False, timeline: bool = False, norm_w: Optional[torch.Tensor] = None,
                 norm_eps: float = 1e-6, add_residual: bool = False):
        self.H, self.I, self.E, self.K = H, I, E, K
        self.types = tuple(types)
        self.max_tokens = max_tokens
        self.router = None if router is None else _need(router, torch.float32, "router")
        self.gate_exps = _need(gate_exps, torch.uint8, "gate_exps")
        self.up_exps = _need(up_exps, torch.uint8, "up_exps")
        self.down_exps = _need(down_exps, torch.uint8, "down_exps")
        self.shared = shared
        d = LayerDesc()
        d.hidden, d.inter, d.n_experts, d.top_k = H, I, E, K
        d.gate_type, d.up_type, d.down_type = self.types
        d.router = _p(self.router)
        d.gate_exps, d.up_exps, d.down_exps = _p(gate_exps), _p(up_exps), _p(down_exps)
        d.gate_stride, d.up_stride, d.down_stride = strides
        d.flags = (_lib.FLAG_MULTI_KERNEL if multi_kernel else 0) | (_lib.FLAG_TIMELINE if timeline else 0)
        if shared is not None:
            for t, n in ((shared.gate, "shared.gate"), (shared.up, "shared.up"), (shared.down, "shared.down")):
                _need(t, torch.uint8, n)
            d.sh_gate, d.sh_up, d.sh_down = _p(shared.gate), _p(shared.up), _p(shared.down)
            d.sh_gate_type, d.sh_up_type, d.sh_down_type = shared.types
            d.inter_shared = shared.inter
            if shared.gate_inp is not None:
                d.sh_gate_inp = _p(_need(shared.gate_inp, torch.float32, "shared.gate_inp"))
        # the step either side: decode(h) normalises h itself (attention.h:29-44)
        # and, with add_residual, returns h + moe_out (winmoe_inference.c:2041)
        self.norm_w = None if norm_w is None else _need(norm_w, torch.float32, "norm_w")
        if self.norm_w is not None and self.norm_w.numel() != H:
            raise ValueError(f"norm_w must hold H = {H} values, got {self.norm_w.numel()}")
        d.norm_w = _p(self.norm_w)
        d.norm_eps = norm_eps
        d.add_residual = 1 if add_residual else 0
        self.desc = d
        L = load()
        nbytes = L.wm_workspace_size(C.byref(d), max_tokens)
        if nbytes < 0:
            raise ValueError("invalid layer descriptor")
        self.ws = _ws(nbytes, gate_exps.device)
        self.step = 0
        self.reset()
        io, wo, ho = C.c_int64(), C.c_int64(), C.c_int64()
        check(L.wm_workspace_trace(C.byref(d), max_tokens, C.byref(io), C.byref(wo), C.byref(ho)), "trace")
        self._trace_off = (io.value, wo.value, ho.value)

    def _need_vec(self, x: torch.Tensor, out: Optional[torch.Tensor]) -> None:
        """x (and out, when given) must be fp32 vectors of H values on the device."""
        _need(x, torch.float32, "x")
        if x.numel() != self.H:
            raise ValueError(f"x must hold H = {self.H} values, got {x.numel()}")
        if out is not None:
            _need(out, torch.float32, "out")
            if out.numel() != self.H:
                raise ValueError(f"out must hold H = {self.H} values, got {out.numel()}")

    def reset(self, stream=None) -> None:
        """Clear the routing trace, hit counters and status bits."""
        check(load().wm_workspace_reset(C.byref(self.desc), self.max_tokens, _p(self.ws), self.ws.numel(),
                                        _stream(stream)), "wm_workspace_reset")
        self.step = 0

    def decode(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, step: Optional[int] = None,
               stream=None) -> torch.Tensor:
        """One token through the layer; routing recorded in the trace.

        Returns moe_out (the layer output before the residual add), or, when
        the layer was built with ``add_residual=True``, ``h + moe_out`` where x
        is the residual stream h.  With ``norm_w`` the layer normalises x
        itself before routing (RMSNorm, attention.h:29-44)."""
        self._need_vec(x, out)
        if out is None:
            out = torch.empty(self.H, dtype=torch.float32, device=x.device)
        st = self.step if step is None else step
        check(load().wm_moe_decode(C.byref(self.desc), _p(x), _p(out), _p(self.ws), self.ws.numel(),
                                   self.max_tokens, st, _stream(stream)), "wm_moe_decode")
        self.step = st + 1
        return out

    def decode_forced(self, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None,
                      step: Optional[int] = None, stream=None) -> torch.Tensor:
        """One token with caller-supplied routing (ids int32[K], w fp32[K] on
        device); the output is as for ``decode``."""
        self._need_vec(x, out)
        _need(ids, torch.int32, "ids")
        _need(w, torch.float32, "w")
        if ids.numel() != self.K or w.numel() != self.K:
            raise ValueError(f"ids and w must hold K = {self.K} values")
        if out is None:
            out = torch.empty(self.H, dtype=torch.float32, device=x.device)
        st = self.step if step is None else step
        check(load().wm_moe_decode_forced(C.byref(self.desc), _p(x), _p(ids), _p(w), _p(out), _p(self.ws),
                                          self.ws.numel(), self.max_tokens, st, _stream(stream)),
              "wm_moe_decode_forced")
        self.step = st + 1
        return out

    def _prefill_ws(self, T: int) -> torch.Tensor:
        """The prefill workspace (allocated on first use, sized for max(T, max_tokens))."""
        need_tokens = max(T, self.max_tokens)
        if getattr(self, "pf_ws", None) is None or self.pf_tokens < need_tokens:
            nbytes = load().wm_prefill_workspace_size(C.byref(self.desc), need_tokens)
            if nbytes < 0:
                raise ValueError("invalid layer descriptor for prefill")
            self.pf_ws = _ws(nbytes, self.gate_exps.device)
            self.pf_ws.zero_()
            self.pf_tokens = need_tokens
        return self.pf_ws

    def prefill(self, x_bf16: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """moe_out for T prompt tokens (x bf16 [T][H]) -> fp32 [T][H], routed by the router."""
        _need(x_bf16, torch.bfloat16, "x")
        T = x_bf16.shape[0]
        if out is None:
            out = torch.empty(T, self.H, dtype=torch.float32, device=x_bf16.device)
        ws = self._prefill_ws(T)
        check(load().wm_moe_prefill(C.byref(self.desc), _p(x_bf16), T, _p(out), _p(ws), ws.numel(), self.pf_tokens,
                                    _stream(stream)), "wm_moe_prefill")
        return out

    def prefill_forced(self, x_bf16: torch.Tensor, ids: torch.Tensor, w: torch.Tensor,
                       out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """Prefill with caller routing: ids int32 [T][K], w fp32 [T][K] on device."""
        _need(x_bf16, torch.bfloat16, "x")
        _need(ids, torch.int32, "ids")
        _need(w, torch.float32, "w")
        T = x_bf16.shape[0]
        if ids.shape != (T, self.K) or w.shape != (T, self.K):
            raise ValueError("ids / w must be [T][K]")
        if out is None:
            out = torch.empty(T, self.H, dtype=torch.float32, device=x_bf16.device)
        ws = self._prefill_ws(T)
        check(load().wm_moe_prefill_forced(C.byref(self.desc), _p(x_bf16), T, _p(ids), _p(w), _p(out), _p(ws),
                                           ws.numel(), self.pf_tokens, _stream(stream)), "wm_moe_prefill_forced")
        return out

    def prefill_status(self) -> int:
        """Status bits of the prefill workspace (synchronises the host)."""
        v = C.c_int32()
        check(load().wm_workspace_status(_p(self.pf_ws), self.pf_ws.numel(), C.byref(v)), "wm_workspace_status")
        return v.value

    def prefill_routing(self, T: int):
        """(ids int32 [T][K], weights fp32 [T][K]) of the last prefill call."""
        io, wo, ho = C.c_int64(), C.c_int64(), C.c_int64()
        check(load().wm_prefill_workspace_routing(C.byref(self.desc), self.pf_tokens, C.byref(io), C.byref(wo),
                                                  C.byref(ho)), "wm_prefill_workspace_routing")
        n = T * self.K * 4
        ids = self.pf_ws[io.value:io.value + n].view(torch.int32).view(T, self.K)
        w = self.pf_ws[wo.value:wo.value + n].view(torch.float32).view(T, self.K)
        return ids, w

    # -- trace ---------------------------------------------------------------
    def trace(self, check: bool = True):
        """(ids int32 [max_tokens][K], weights fp32 [max_tokens][K]) views of
        the device trace.  With ``check`` (the default) the queued steps are
        waited for and a step that gave up raises (see ``check()``)."""
        if check:
            self.check()
        io, wo, _ = self._trace_off
        n = self.max_tokens * self.K * 4
        ids = self.ws[io:io + n].view(torch.int32).view(self.max_tokens, self.K)
        w = self.ws[wo:wo + n].view(torch.float32).view(self.max_tokens, self.K)
        return ids, w

    def hits(self) -> torch.Tensor:
        """Per-expert selection counters (uint32 stored, returned as int32 view)."""
        _, _, ho = self._trace_off
        return self.ws[ho:ho + self.E * 4].view(torch.int32)

    def timeline(self):
        """Per-work-item timeline of the last fused step: uint64 [items][8]
        (start, dependencies met, main work done, end in device clock ticks;
        kind | hw ids; three zero words)."""
        off, cap = C.c_int64(), C.c_int64()
        check(load().wm_workspace_timeline(C.byref(self.desc), self.max_tokens, C.byref(off), C.byref(cap)),
              "wm_workspace_timeline")
        n = cap.value * 8 * 8
        return self.ws[off.value:off.value + n].view(torch.int64).view(cap.value, 8)

    def check(self) -> int:
        """Waits for the layer's queued work and returns its status bits;
        raises WinMoEError when a decode step gave up waiting
        (WM_STATUS_SPIN_TIMEOUT: its outputs are invalid, ``reset()`` before
        the next call).  The other bits describe the routing, not a failure."""
        st = self.status()
        if st & _lib.STATUS_SPIN_TIMEOUT:
            raise _lib.WinMoEError("a decode step gave up waiting for another workgroup (WM_STATUS_SPIN_TIMEOUT): "
                                   "its outputs are invalid; reset() the layer", _lib.WM_ERR)
        return st

    def status(self) -> int:
        """Status bits of the decode workspace (synchronises the host)."""
        v = C.c_int32()
        check(load().wm_workspace_status(_p(self.ws), self.ws.numel(), C.byref(v)), "wm_workspace_status")
        return v.value


def decode_stack(layers, x: torch.Tensor, out: Optional[torch.Tensor] = None, routes=None,
                 step: Optional[int] = None, stream=None) -> torch.Tensor:
    """One token through a chain of layers (wm_moe_decode_stack): layer l's
    input is layer l-1's output (x for the first), so with each layer's
    RMSNorm and residual add out[l] = h_{l+1} = h_l + moe_l(rmsnorm(h_l)).
    Up to 8 layers run in one launch.  routes: None (every layer routed by
    its router) or one (ids int32[K], w fp32[K]) device pair per layer (None
    entries: that layer's router).  Returns out fp32 [n_layers][H], each
    layer's output, bit for bit what the layers' own decode calls give."""
    n = len(layers)
    if n == 0:
        raise ValueError("no layers")
    L0 = layers[0]
    for m in layers:
        if m.H != L0.H or m.max_tokens != L0.max_tokens:
            raise ValueError("the layers of a chain share the hidden size and max_tokens")
    L0._need_vec(x, None)
    if out is None:
        out = torch.empty(n, L0.H, dtype=torch.float32, device=x.device)
    _need(out, torch.float32, "out")
    if out.shape != (n, L0.H) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous [{n}][{L0.H}] tensor")
    st = L0.step if step is None else step
    descs = (C.c_void_p * n)(*[C.cast(C.pointer(m.desc), C.c_void_p) for m in layers])
    wss = (C.c_void_p * n)(*[m.ws.data_ptr() for m in layers])
    wsb = (C.c_int64 * n)(*[m.ws.numel() for m in layers])
    ids_arr = w_arr = None
    if routes is not None:
        if len(routes) != n:
            raise ValueError("routes: one entry per layer")
        pi, pw = [], []
        for m, r in zip(layers, routes):
            if r is None:
                pi.append(None)
                pw.append(None)
                continue
            ids, w = r
            _need(ids, torch.int32, "ids")
            _need(w, torch.float32, "w")
            if ids.numel() != m.K or w.numel() != m.K:
                raise ValueError(f"ids and w must hold K = {m.K} values")
            pi.append(ids.data_ptr())
            pw.append(w.data_ptr())
        ids_arr = (C.c_void_p * n)(*pi)
        w_arr = (C.c_void_p * n)(*pw)
    check(load().wm_moe_decode_stack(n, descs, wss, wsb, _p(x), _p(out), ids_arr, w_arr, L0.max_tokens, st,
                                     _stream(stream)), "wm_moe_decode_stack")
    for m in layers:
        m.step = st + 1
    return out


class ExpertPool:
    """Host -> HBM expert streaming (include/winmoe_hip.h, wm_pool_*): ``n_slots``
    expert slots in HBM filled on demand from host memory, for models whose
    experts do not all fit there (the reference's miss path,
    winmoe_inference.c:1736-1789, and GPU cache upload,
    gpu_offload.cu:590-659).  ``layer(...)`` builds a MoELayer whose expert
    tensors are the slots; a step on it runs ``decode_forced`` with the slot
    indices ``acquire`` returns.  Host tensors should be pinned
    (``pin_memory=True``) for the copies to overlap compute."""

    def __init__(self, n_slots: int, gate_bytes: int, up_bytes: int, down_bytes: int, device="cuda"):
        L = load()
        sb = L.wm_pool_slot_bytes(gate_bytes, up_bytes, down_bytes)
        if sb < 0:
            raise ValueError("expert part sizes must be positive")
        self.n_slots, self.slot_bytes = n_slots, sb
        self.parts = (gate_bytes, up_bytes, down_bytes)
        g256 = (gate_bytes + 255) // 256 * 256
        self.offsets = (0, g256, g256 + (up_bytes + 255) // 256 * 256)
        self.mem = _ws(n_slots * sb, device)
        h = C.c_void_p()
        check(L.wm_pool_create(_p(self.mem), self.mem.numel(), n_slots, gate_bytes, up_bytes, down_bytes,
                               C.byref(h)), "wm_pool_create")
        self._h = h
        self.slots = torch.zeros(n_slots, dtype=torch.int32, device=device)

    def layer(self, H: int, I: int, K: int, types: Sequence[int], shared: Optional[SharedExpert] = None,
              max_tokens: int = 256, **kw) -> "MoELayer":
        """A layer whose routed experts are the pool's slots (no router: its
        steps take slot indices through ``decode_forced``)."""
        views = [self.mem[o:] for o in self.offsets]
        return MoELayer(H, I, self.n_slots, K, None, views[0], views[1], views[2], types, shared=shared,
                        max_tokens=max_tokens, strides=(self.slot_bytes,) * 3, **kw)

    def _ids(self, ids, n_src: int) -> np.ndarray:
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32).reshape(-1))
        if ids.size and (ids.min() < 0 or ids.max() >= n_src):
            raise ValueError(f"expert ids must lie in [0, {n_src}) (the host source's experts)")
        return ids

    def acquire(self, layer: int, ids, gate_src: torch.Tensor, up_src: torch.Tensor, down_src: torch.Tensor,
                out: Optional[torch.Tensor] = None, stream=None):
        """Makes experts ``ids`` of ``layer`` resident (copies the missing ones
        from the host tensors ``*_src`` [E][bytes], three copies per expert);
        returns (slots, misses): the device int32 slot indices, written in
        stream order, and the miss count."""
        for t, n in ((gate_src, "gate_src"), (up_src, "up_src"), (down_src, "down_src")):
            if t.device.type != "cpu" or t.dtype != torch.uint8 or t.dim() != 2 or not t.is_contiguous():
                raise ValueError(f"{n} must be a contiguous uint8 host tensor [E][bytes]")
        n_src = gate_src.shape[0]
        if up_src.shape[0] != n_src or down_src.shape[0] != n_src:
            raise ValueError("gate_src, up_src and down_src must hold the same experts")
        ids = self._ids(ids, n_src)
        if out is None:
            out = torch.empty(ids.size, dtype=torch.int32, device=self.mem.device)
        rc = load().wm_pool_acquire(self._h, layer, ids.ctypes.data_as(C.POINTER(C.c_int32)), ids.size, n_src,
                                    gate_src.data_ptr(), up_src.data_ptr(), down_src.data_ptr(),
                                    gate_src.stride(0), up_src.stride(0), down_src.stride(0), _p(out),
                                    _stream(stream))
        if rc < 0:
            check(rc, "wm_pool_acquire")
        return out, rc

    def pack(self, gate_src: torch.Tensor, up_src: torch.Tensor, down_src: torch.Tensor,
             pin: bool = True) -> torch.Tensor:
        """Host tensor [E][slot_bytes] holding each expert as one slot image
        ([gate | up | down] at the slot's 256-byte aligned part offsets), the
        source of ``acquire_packed``."""
        E = gate_src.shape[0]
        out = torch.zeros((E, self.slot_bytes), dtype=torch.uint8, pin_memory=pin)
        for o, t, nb in zip(self.offsets, (gate_src, up_src, down_src), self.parts):
            out[:, o:o + nb] = t[:, :nb]
        return out

    def acquire_packed(self, layer: int, ids, src: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None):
        """As ``acquire``, from slot images (``pack``): one copy per missing expert."""
        if src.device.type != "cpu" or src.dtype != torch.uint8 or src.dim() != 2 or not src.is_contiguous():
            raise ValueError("src must be a contiguous uint8 host tensor [E][slot_bytes]")
        ids = self._ids(ids, src.shape[0])
        if out is None:
            out = torch.empty(ids.size, dtype=torch.int32, device=self.mem.device)
        rc = load().wm_pool_acquire_packed(self._h, layer, ids.ctypes.data_as(C.POINTER(C.c_int32)), ids.size,
                                           src.shape[0], src.data_ptr(), src.stride(0), _p(out), _stream(stream))
        if rc < 0:
            check(rc, "wm_pool_acquire_packed")
        return out, rc

    def release(self, stream=None) -> None:
        """After the steps that read the acquired slots are enqueued on ``stream``."""
        check(load().wm_pool_release(self._h, _stream(stream)), "wm_pool_release")

    def stats(self):
        """(hits, misses, bytes copied) since creation."""
        h, m, b = C.c_int64(), C.c_int64(), C.c_int64()
        check(load().wm_pool_stats(self._h, C.byref(h), C.byref(m), C.byref(b)), "wm_pool_stats")
        return h.value, m.value, b.value

    def close(self) -> None:
        if self._h:
            load().wm_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
