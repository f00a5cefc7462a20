"""ctypes access to the CPU oracle (liboracle.so) and the reference build (_ref/libwmref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg, as the parity reference.  The product package never imports
this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libwmref.so")

F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 8, 10, 11, 12, 13, 14
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}

_fp = C.POINTER(C.c_float)
_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int32)
_vp = C.c_void_p


class WmoLayer(C.Structure):
    """Mirror of ``wmo_layer`` in wm_oracle.h."""
    _fields_ = [
        ("H", C.c_int32), ("I", C.c_int32), ("I_shared", C.c_int32), ("E", C.c_int32), ("K", C.c_int32),
        ("gate_type", C.c_int32), ("up_type", C.c_int32), ("down_type", C.c_int32),
        ("sh_gate_type", C.c_int32), ("sh_up_type", C.c_int32), ("sh_down_type", C.c_int32),
        ("router", _vp), ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
        ("gate_stride", C.c_int64), ("up_stride", C.c_int64), ("down_stride", C.c_int64),
        ("sh_gate", _vp), ("sh_up", _vp), ("sh_down", _vp), ("sh_gate_inp", _vp),
    ]


def build():
    """Compile liboracle.so (and _ref when the reference sources are present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray, t=_vp):
    if t is _vp:
        return a.ctypes.data_as(_vp)
    return a.ctypes.data_as(t)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = C.CDLL(ORACLE_SO)
        L.wmo_fp16_to_fp32.restype = C.c_float
        L.wmo_fp16_to_fp32.argtypes = [C.c_uint16]
        L.wmo_dequant.argtypes = [C.c_int, _vp, C.c_int64, _fp]
        L.wmo_dequant_block_sums.argtypes = [C.c_int, _vp, C.c_int64, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
        L.wmo_router_logits.argtypes = [_fp, _fp, C.c_int, C.c_int, _fp]
        L.wmo_topk_softmax.argtypes = [_fp, C.c_int, C.c_int, _ip, _fp]
        L.wmo_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        L.wmo_sigmoid.restype = C.c_double
        L.wmo_sigmoid.argtypes = [C.c_double]
        L.wmo_matvec.argtypes = [C.c_int, _vp, _dp, C.c_int, C.c_int, _dp]
        L.wmo_expert_ffn.argtypes = [_vp, C.c_int, _vp, C.c_int, _vp, C.c_int, _dp, C.c_int, C.c_int, _dp, _dp]
        L.wmo_moe_layer.argtypes = [C.POINTER(WmoLayer), _fp, _ip, _fp, _ip, _fp, _dp]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    """The reference's own kernels compiled from source (None if not built)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_SO):
            return None
        R = C.CDLL(REF_SO)
        R.ref_cpu_supported.restype = C.c_int
        if not R.ref_cpu_supported():
            return None
        R.ref_fp16_to_fp32.restype = C.c_float
        R.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        R.ref_q8_dequant_row.argtypes = [_vp, C.c_int, _fp]
        for n in ("ref_q6k_dot_block", "ref_q6k_dot_block_avx2", "ref_q4k_dot_q8k", "ref_q5k_dot_q8k",
                  "ref_q8_dot_block"):
            getattr(R, n).restype = C.c_float
            getattr(R, n).argtypes = [_vp, _fp]
        R.ref_decode_q4k_scales.argtypes = [_vp, _vp, _vp]
        R.ref_quantize_row_q8_K.argtypes = [_fp, C.c_int, _vp]
        R.ref_sigmoid_stable.restype = C.c_float
        R.ref_sigmoid_stable.argtypes = [C.c_float]
        R.ref_router_topk.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_int, _ip, _fp]
        R.ref_moe_layer_cpu.argtypes = [C.POINTER(WmoLayer), _fp, _ip, _fp, _ip, _fp, _fp]
        R.wmref_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int]
        _ref = R
    return _ref


# ---------------------------------------------------------------- wrappers

def fp16_to_fp32(h: int) -> float:
    return lib().wmo_fp16_to_fp32(h)


def dequant(qtype: int, blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    bs = BLOCK_BYTES[qtype]
    assert b.size % bs == 0
    nb = b.size // bs
    out = np.empty(nb * BLOCK_ELEMS[qtype], dtype=np.float32)
    rc = lib().wmo_dequant(qtype, _ptr(b), nb, _ptr(out, _fp))
    assert rc == 0, rc
    return out


def dequant_block_sums(qtype: int, blocks: np.ndarray, threads: int = 1):
    """Per-block checksums of the dequantised weights (wmo_dequant_block_sums):
    s1[i] = sum over block i of the values' fp32 bit patterns (unsigned),
    s2[i] = the same weighted by position + 1.  `threads` workers split the
    blocks (the C call releases the GIL)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    bs = BLOCK_BYTES[qtype]
    assert b.size % bs == 0
    nb = b.size // bs
    s1 = np.empty(nb, np.int64)
    s2 = np.empty(nb, np.int64)
    L = lib()
    _i64 = C.POINTER(C.c_int64)

    def part(r):
        i0, i1 = r
        if i1 <= i0:
            return 0
        return L.wmo_dequant_block_sums(qtype, b.ctypes.data + i0 * bs, i1 - i0,
                                        C.cast(s1.ctypes.data + 8 * i0, _i64), C.cast(s2.ctypes.data + 8 * i0, _i64))

    n = max(1, int(threads))
    step = (nb + n - 1) // n
    ranges = [(i, min(nb, i + step)) for i in range(0, nb, step)] or [(0, 0)]
    if n == 1 or len(ranges) == 1:
        rcs = [part(r) for r in ranges]
    else:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=n) as ex:
            rcs = list(ex.map(part, ranges))
    assert all(rc == 0 for rc in rcs), rcs
    return s1, s2


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """attention.h:29-44 (wmo_rmsnorm)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().wmo_rmsnorm(_ptr(out, _fp), _ptr(x, _fp), _ptr(w, _fp), x.shape[0], eps)
    return out


def ref_rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The reference's rmsnorm (attention.h:29-44, eps 1e-6) compiled from its
    sources; the oracle's restatement when that build is absent."""
    R = ref()
    if R is None:
        return rmsnorm(x, w)
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    R.wmref_rmsnorm(_ptr(out, _fp), _ptr(x, _fp), _ptr(w, _fp), x.shape[0])
    return out


def router_logits(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    E, H = W.shape
    out = np.empty(E, np.float32)
    lib().wmo_router_logits(_ptr(x, _fp), _ptr(W, _fp), H, E, _ptr(out, _fp))
    return out


def topk_softmax(logits: np.ndarray, K: int):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    deg = lib().wmo_topk_softmax(_ptr(lg, _fp), lg.size, K, _ptr(ids, _ip), _ptr(w, _fp))
    return ids, w, deg


def router_topk(x, W, K):
    return topk_softmax(router_logits(x, W), K)


def matvec(qtype, W: np.ndarray, x: np.ndarray, rows: int, inp: int) -> np.ndarray:
    Wb = np.ascontiguousarray(W, np.uint8).reshape(-1)
    xd = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    rc = lib().wmo_matvec(qtype, _ptr(Wb), _ptr(xd, _dp), rows, inp, _ptr(y, _dp))
    assert rc == 0, rc
    return y


def expert_ffn(gate, gt, up, ut, down, dt, x, H, I, want_act=False):
    xd = np.ascontiguousarray(x, np.float64)
    y = np.empty(H, np.float64)
    act = np.empty(I, np.float64)
    g = np.ascontiguousarray(gate, np.uint8)
    u = np.ascontiguousarray(up, np.uint8)
    d = np.ascontiguousarray(down, np.uint8)
    rc = lib().wmo_expert_ffn(_ptr(g), gt, _ptr(u), ut, _ptr(d), dt, _ptr(xd, _dp), H, I, _ptr(y, _dp),
                              _ptr(act, _dp))
    assert rc == 0, rc
    return (y, act) if want_act else y


def make_layer(H, I, E, K, types, router=None, gate=None, up=None, down=None, shared=None,
               sh_types=None, sh_gate_inp=None, I_shared=0, strides=(0, 0, 0)):
    """Build a WmoLayer over numpy arrays (kept alive on the returned object)."""
    L = WmoLayer()
    L.H, L.I, L.E, L.K = H, I, E, K
    L.I_shared = I_shared
    L.gate_type, L.up_type, L.down_type = types
    keep = []

    def p(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    L.router = p(None if router is None else np.asarray(router, np.float32))
    L.gate_exps, L.up_exps, L.down_exps = p(gate), p(up), p(down)
    L.gate_stride, L.up_stride, L.down_stride = strides
    if shared is not None:
        L.sh_gate, L.sh_up, L.sh_down = p(shared[0]), p(shared[1]), p(shared[2])
        L.sh_gate_type, L.sh_up_type, L.sh_down_type = sh_types
    L.sh_gate_inp = p(None if sh_gate_inp is None else np.asarray(sh_gate_inp, np.float32))
    L._keep = keep
    return L


def moe_layer(L: WmoLayer, x: np.ndarray, forced_ids=None, forced_w=None):
    xf = np.ascontiguousarray(x, np.float32)
    ids = np.empty(L.K, np.int32)
    w = np.empty(L.K, np.float32)
    out = np.empty(L.H, np.float64)
    fi = None if forced_ids is None else np.ascontiguousarray(forced_ids, np.int32)
    fw = None if forced_w is None else np.ascontiguousarray(forced_w, np.float32)
    rc = lib().wmo_moe_layer(C.byref(L), _ptr(xf, _fp), None if fi is None else _ptr(fi, _ip),
                             None if fw is None else _ptr(fw, _fp), _ptr(ids, _ip), _ptr(w, _fp),
                             _ptr(out, _dp))
    assert rc >= 0, rc
    return ids, w, out, rc


def ref_moe_layer_cpu(L: WmoLayer, x: np.ndarray, forced_ids=None, forced_w=None):
    """Reference CPU path (compiled from the reference headers); None if unavailable."""
    R = ref()
    if R is None:
        return None
    xf = np.ascontiguousarray(x, np.float32)
    ids = np.empty(L.K, np.int32)
    w = np.empty(L.K, np.float32)
    out = np.empty(L.H, np.float32)
    fi = None if forced_ids is None else np.ascontiguousarray(forced_ids, np.int32)
    fw = None if forced_w is None else np.ascontiguousarray(forced_w, np.float32)
    rc = R.ref_moe_layer_cpu(C.byref(L), _ptr(xf, _fp), None if fi is None else _ptr(fi, _ip),
                             None if fw is None else _ptr(fw, _fp), _ptr(ids, _ip), _ptr(w, _fp),
                             _ptr(out, _fp))
    assert rc >= 0, rc
    return ids, w, out, rc
