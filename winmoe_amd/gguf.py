"""GGUF v3 reader / writer and the MoE-layer slicer: the input side of the boundary.

Restates the container that engine/runtime/gguf_parser.h reads (``parse_gguf``
:149-244, ``parse_gguf_split`` :252-347, ``find_tensor`` :350-358, type tables
:21-57) from the published GGUF v3 layout, without that parser's faults:

* every ggml block type has its block size (Q8_0 34 B / 32, Q2_K 84 / 256,
  Q3_K 110 / 256, ...), so a stacked expert tensor's byte size -- and with it
  the per-expert stride ``nbytes / E`` (winmoe_inference.c:467-489) -- is right
  for every expert type;
* every metadata value is skipped by its real size (bool 1 byte, uint64 /
  int64 / float64 8 bytes, strings and arrays by their lengths);
* the tensor data starts at the ``general.alignment`` boundary (32 when the
  key is absent), and each tensor's offset is checked against it.

Files are memory-mapped; nothing is read until a tensor's bytes are asked for.
``moe_layer_from_gguf`` maps one layer's router, stacked experts and shared
expert into HBM once and returns a :class:`MoELayer` over them.
"""
from __future__ import annotations

import os
import re
import struct
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types (GGUF v3)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# ggml tensor types: (elements per block, bytes per block)
GGML_BLOCK = {
    0: (1, 4),       # F32
    1: (1, 2),       # F16
    2: (32, 18),     # Q4_0
    3: (32, 20),     # Q4_1
    6: (32, 22),     # Q5_0
    7: (32, 24),     # Q5_1
    8: (32, 34),     # Q8_0
    9: (32, 36),     # Q8_1
    10: (256, 84),   # Q2_K
    11: (256, 110),  # Q3_K
    12: (256, 144),  # Q4_K
    13: (256, 176),  # Q5_K
    14: (256, 210),  # Q6_K
    15: (256, 292),  # Q8_K
    24: (1, 1),      # I8
    25: (1, 2),      # I16
    26: (1, 4),      # I32
    27: (1, 8),      # I64
    28: (1, 8),      # F64
    30: (1, 2),      # BF16
}


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file."""


@dataclass
class Value:
    """A metadata value with its GGUF type (arrays: ``elem`` is the element type)."""
    type: int
    value: object
    elem: Optional[int] = None


@dataclass
class Tensor:
    name: str
    dims: Tuple[int, ...]       # ne0 first (ne0 is the contiguous dimension)
    ggml_type: int
    offset: int                 # from the start of its file's data section
    nbytes: int
    shard: int                  # index of the file that holds it

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


def tensor_nbytes(dims: Sequence[int], ggml_type: int) -> int:
    if ggml_type not in GGML_BLOCK:
        raise GGUFError(f"unknown ggml type {ggml_type}")
    be, bb = GGML_BLOCK[ggml_type]
    n = 1
    for d in dims:
        n *= int(d)
    if dims and dims[0] % be:
        raise GGUFError(f"row length {dims[0]} is not a multiple of the {be}-element block of type {ggml_type}")
    return n // be * bb


class _Reader:
    def __init__(self, buf: memoryview, name: str):
        self.b, self.p, self.name = buf, 0, name

    def take(self, n: int) -> memoryview:
        if n < 0 or self.p + n > len(self.b):
            raise GGUFError(f"{self.name}: truncated at byte {self.p} (need {n} more)")
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(UINT64)
        return bytes(self.take(n)).decode("utf-8")

    def value(self, t: int) -> Value:
        if t in _SCALAR:
            return Value(t, self.scalar(t))
        if t == STRING:
            return Value(t, self.string())
        if t == ARRAY:
            et = self.scalar(UINT32)
            n = self.scalar(UINT64)
            if et == ARRAY:
                return Value(t, [self.value(ARRAY) for _ in range(n)], ARRAY)
            if et == STRING:
                return Value(t, [self.string() for _ in range(n)], STRING)
            if et not in _SCALAR:
                raise GGUFError(f"{self.name}: unknown array element type {et}")
            fmt = _SCALAR[et]
            sz = struct.calcsize(fmt)
            raw = self.take(n * sz)
            return Value(t, [struct.unpack_from(fmt, raw, i * sz)[0] for i in range(n)], et)
        raise GGUFError(f"{self.name}: unknown metadata value type {t}")


class GGUFFile:
    """One GGUF model, possibly split over several shard files
    (``name-00001-of-0000N.gguf``; gguf_parser.h:252-347).  ``kv`` holds the
    first shard's metadata (plain Python values; ``kv_typed`` keeps the GGUF
    types), ``tensors`` every shard's tensors by name."""

    def __init__(self, path: str):
        paths = _shard_paths(path)
        self.paths = paths
        self._maps: List[np.memmap] = []
        self._data_start: List[int] = []
        self.tensors: Dict[str, Tensor] = {}
        self.kv_typed: Dict[str, Value] = {}
        for i, p in enumerate(paths):
            kv, tensors, start = self._parse(p, i)
            if i == 0:
                self.kv_typed = kv
            for t in tensors:
                if t.name in self.tensors:
                    raise GGUFError(f"tensor {t.name} appears twice")
                self.tensors[t.name] = t
            self._data_start.append(start)
        self.kv = {k: v.value for k, v in self.kv_typed.items()}
        self.alignment = int(self.kv.get("general.alignment", DEFAULT_ALIGNMENT))

    def _parse(self, path: str, shard: int):
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        self._maps.append(mm)
        r = _Reader(memoryview(mm), os.path.basename(path))
        if bytes(r.take(4)) != MAGIC:
            raise GGUFError(f"{path}: not a GGUF file")
        version = r.scalar(UINT32)
        if version not in (2, 3):
            raise GGUFError(f"{path}: GGUF version {version} is not supported (2 and 3 are)")
        n_tensors = r.scalar(UINT64)
        n_kv = r.scalar(UINT64)
        kv: Dict[str, Value] = {}
        for _ in range(n_kv):
            key = r.string()
            kv[key] = r.value(r.scalar(UINT32))
        align = int(kv["general.alignment"].value) if "general.alignment" in kv else DEFAULT_ALIGNMENT
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{path}: general.alignment {align} is not a power of two")
        tensors = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar(UINT32)
            dims = tuple(r.scalar(UINT64) for _ in range(nd))
            gt = r.scalar(UINT32)
            off = r.scalar(UINT64)
            if off % align:
                raise GGUFError(f"{path}: tensor {name} offset {off} is not {align}-aligned")
            tensors.append(Tensor(name, dims, gt, off, tensor_nbytes(dims, gt), shard))
        start = (r.p + align - 1) // align * align
        for t in tensors:
            if start + t.offset + t.nbytes > len(mm):
                raise GGUFError(f"{path}: tensor {t.name} runs past the end of the file")
        return kv, tensors, start

    def find(self, name: str) -> Optional[Tensor]:
        """The tensor called ``name``, or None (gguf_parser.h:350-358)."""
        return self.tensors.get(name)

    def data(self, name: str) -> np.ndarray:
        """The raw bytes of a tensor (a read-only view of the mapped file)."""
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(name)
        s = self._data_start[t.shard] + t.offset
        return self._maps[t.shard][s:s + t.nbytes]

    def arch(self) -> str:
        return str(self.kv.get("general.architecture", ""))


def _shard_paths(path: str) -> List[str]:
    m = re.match(r"^(.*)-(\d{5})-of-(\d{5})\.gguf$", path)
    if not m:
        return [path]
    n = int(m.group(3))
    return [f"{m.group(1)}-{i:05d}-of-{n:05d}.gguf" for i in range(1, n + 1)]


# ------------------------------------------------------------------ writer

def _pack_value(v: Value) -> bytes:
    if v.type in _SCALAR:
        return struct.pack(_SCALAR[v.type], v.value)
    if v.type == STRING:
        b = str(v.value).encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if v.type == ARRAY:
        et = v.elem
        items = list(v.value)
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _pack_value(it if isinstance(it, Value) else Value(et, it))
        return out
    raise GGUFError(f"unknown metadata value type {v.type}")


def _as_value(v) -> Value:
    if isinstance(v, Value):
        return v
    if isinstance(v, bool):
        return Value(BOOL, v)
    if isinstance(v, int):
        return Value(UINT32 if 0 <= v < 2 ** 32 else INT64, v)
    if isinstance(v, float):
        return Value(FLOAT32, v)
    if isinstance(v, str):
        return Value(STRING, v)
    raise GGUFError(f"no GGUF type for {v!r}; wrap it in Value")


def write_gguf(path: str, kv: Dict[str, object], tensors: Sequence[Tuple[str, Sequence[int], int, bytes]],
               alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Write a GGUF file: ``tensors`` are (name, dims ne0-first, ggml type, raw bytes).
    A ``general.alignment`` other than 32 is written into the metadata."""
    kv = dict(kv)
    if alignment != DEFAULT_ALIGNMENT:
        kv["general.alignment"] = Value(UINT32, alignment)
    head = MAGIC + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, v in kv.items():
        v = _as_value(v)
        kb = k.encode("utf-8")
        head += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", v.type) + _pack_value(v)
    off = 0
    infos = b""
    offsets = []
    for name, dims, gt, data in tensors:
        n = tensor_nbytes(dims, gt)
        if len(data) != n:
            raise GGUFError(f"tensor {name}: {len(data)} bytes given, {n} expected")
        nb = name.encode("utf-8")
        infos += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        infos += b"".join(struct.pack("<Q", int(d)) for d in dims) + struct.pack("<IQ", gt, off)
        offsets.append(off)
        off = (off + n + alignment - 1) // alignment * alignment
    head += infos
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, dims, gt, data), o in zip(tensors, offsets):
            cur = f.tell() - len(head) - pad
            f.write(b"\0" * (o - cur))
            f.write(bytes(data))


# ------------------------------------------------------------------ MoE layer slicer

def expert_slice(g: GGUFFile, name: str, e: int) -> np.ndarray:
    """Expert e's bytes of a stacked expert tensor: stride = nbytes / E
    (winmoe_inference.c:467-489, 1770-1775), E = the last dimension."""
    t = g.find(name)
    if t is None:
        raise KeyError(name)
    E = t.dims[-1]
    if t.nbytes % E:
        raise GGUFError(f"{name}: {t.nbytes} bytes do not split into {E} experts")
    stride = t.nbytes // E
    if not 0 <= e < E:
        raise IndexError(e)
    return g.data(name)[e * stride:(e + 1) * stride]


def _router_fp32(g: "GGUFFile", name: str, t, E: int, H: int, device) -> torch.Tensor:
    """The router as fp32 [E][H] on the device.  F32 is taken as is; F16 is
    widened exactly; quantised routers (Q8_0, Q2_K .. Q6_K) are dequantised
    exactly by the library.  The reference dispatches a quantised router
    through quant_matvec (transformer.h:120-123), whose Q8_0 / K-quant paths
    round the activations to int8 first, so its logits for such a router can
    differ from the fp32 logits of the dequantised weights in the last bits."""
    import torch

    from . import _lib
    raw = np.array(g.data(name), copy=True)
    if t.ggml_type == 0:
        w = torch.from_numpy(raw.view(np.float32)).to(device)
    elif t.ggml_type == 1:
        w = torch.from_numpy(raw.view(np.float16).astype(np.float32)).to(device)
    elif t.ggml_type in _lib.QUANT_TYPES:
        from .moe import dequantize
        w = dequantize(torch.from_numpy(raw).to(device), t.ggml_type)
    else:
        raise GGUFError(f"router type {t.ggml_type} is not supported (F32, F16, Q8_0, Q2_K .. Q6_K are)")
    return w.view(E, H).contiguous()


def moe_layer_from_gguf(g: GGUFFile, layer: int, K: Optional[int] = None, device="cuda", max_tokens: int = 256,
                        multi_kernel: bool = False):
    """Map layer ``layer``'s MoE block into HBM once and return a MoELayer.

    Tensors (GGUF names, dims ne0-first): ``blk.L.ffn_gate_inp.weight`` fp32
    [H, E]; ``blk.L.ffn_{gate,up}_exps.weight`` [H, I, E] and
    ``blk.L.ffn_down_exps.weight`` [I, H, E] in one quantised type each;
    optional shared expert ``blk.L.ffn_{gate,up,down}_shexp.weight`` and its
    fp32 gate ``blk.L.ffn_gate_inp_shexp.weight`` [H].  K defaults to the
    model's ``<arch>.expert_used_count``."""
    import torch

    from . import _lib
    from .moe import MoELayer, SharedExpert

    pre = f"blk.{layer}."

    def need(n):
        t = g.find(pre + n)
        if t is None:
            raise GGUFError(f"missing tensor {pre + n}")
        return t

    def dev(n):
        return torch.from_numpy(np.array(g.data(pre + n), copy=True)).to(device)

    tg, tu, td = need("ffn_gate_exps.weight"), need("ffn_up_exps.weight"), need("ffn_down_exps.weight")
    if len(tg.dims) != 3 or tg.dims != tu.dims or len(td.dims) != 3:
        raise GGUFError("stacked expert tensors must be 3-D with equal gate/up shapes")
    H, I, E = tg.dims
    if td.dims != (I, H, E):
        raise GGUFError(f"down experts are {td.dims}, expected {(I, H, E)}")
    types = (tg.ggml_type, tu.ggml_type, td.ggml_type)
    for t in types:
        if t not in _lib.QUANT_TYPES:
            raise GGUFError(f"expert type {t} is not supported (Q8_0, Q2_K .. Q6_K are)")
    if K is None:
        K = int(g.kv.get(f"{g.arch()}.expert_used_count", 0))
        if K <= 0:
            raise GGUFError("no expert_used_count in the metadata: pass K")
    router = None
    tr = g.find(pre + "ffn_gate_inp.weight")
    if tr is not None:
        if tr.dims != (H, E):
            raise GGUFError(f"router must be [{H}, {E}], got {tr.dims}")
        router = _router_fp32(g, pre + "ffn_gate_inp.weight", tr, E, H, device)
    shared = None
    if g.find(pre + "ffn_gate_shexp.weight") is not None:
        sg, su, sd = need("ffn_gate_shexp.weight"), need("ffn_up_shexp.weight"), need("ffn_down_shexp.weight")
        Is = sg.dims[1]
        if sg.dims != (H, Is) or su.dims != (H, Is) or sd.dims != (Is, H):
            raise GGUFError("shared expert shapes do not match the layer")
        gi = None
        if g.find(pre + "ffn_gate_inp_shexp.weight") is not None:
            tgi = need("ffn_gate_inp_shexp.weight")
            if tgi.ggml_type != 0 or tgi.dims != (H,):
                raise GGUFError(f"shared-expert gate must be F32 [{H}]")
            gi = torch.from_numpy(np.array(g.data(pre + "ffn_gate_inp_shexp.weight"), copy=True).view(np.float32)).to(
                device)
        shared = SharedExpert(dev("ffn_gate_shexp.weight"), dev("ffn_up_shexp.weight"), dev("ffn_down_shexp.weight"),
                              (sg.ggml_type, su.ggml_type, sd.ggml_type), gi, Is)
    strides = (tg.nbytes // E, tu.nbytes // E, td.nbytes // E)
    return MoELayer(H, I, E, K, router, dev("ffn_gate_exps.weight"), dev("ffn_up_exps.weight"),
                    dev("ffn_down_exps.weight"), types, shared=shared, max_tokens=max_tokens, strides=strides,
                    multi_kernel=multi_kernel)
