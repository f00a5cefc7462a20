"""ctypes binding of libwinmoe_hip.so (include/winmoe_hip.h).

The library is built in-tree by ``winmoe_amd.build``.  Loading fails loudly
when it is missing: there is no CPU fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libwinmoe_hip.so")

WM_OK, WM_ERR, WM_EINVAL = 0, -1, -2
F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 8, 10, 11, 12, 13, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K",
              Q6_K: "Q6_K"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
QUANT_TYPES = (Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)

STATUS_DEGENERATE_ROUTING = 1
STATUS_BAD_EXPERT_ID = 2
STATUS_NONFINITE_WEIGHT = 4
STATUS_SPIN_TIMEOUT = 8
FLAG_MULTI_KERNEL = 1
FLAG_TIMELINE = 2
FLAG_ITEM_KERNEL = 4
FLAG_PERSIST_KERNEL = 8
FLAG_SPIN_PROBE = 16
FLAG_PREFILL_PASS16 = 32
FLAG_PREFILL_PASS32 = 64

_vp, _i64 = C.c_void_p, C.c_int64


class LayerDesc(C.Structure):
    """Mirror of ``wm_layer_desc``."""
    _fields_ = [
        ("hidden", C.c_int32), ("inter", C.c_int32), ("inter_shared", C.c_int32), ("n_experts", C.c_int32),
        ("top_k", C.c_int32), ("gate_type", C.c_int32), ("up_type", C.c_int32), ("down_type", C.c_int32),
        ("sh_gate_type", C.c_int32), ("sh_up_type", C.c_int32), ("sh_down_type", C.c_int32),
        ("flags", C.c_int32),
        ("router", _vp), ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
        ("gate_stride", _i64), ("up_stride", _i64), ("down_stride", _i64),
        ("sh_gate", _vp), ("sh_up", _vp), ("sh_down", _vp), ("sh_gate_inp", _vp),
        ("norm_w", _vp), ("norm_eps", C.c_float), ("add_residual", C.c_int32),
    ]


# name -> (restype, argtypes); every symbol include/winmoe_hip.h declares.
SIGNATURES = {
    "wm_init": (C.c_int, []),
    "wm_version": (C.c_char_p, []),
    "wm_block_bytes": (C.c_int, [C.c_int]),
    "wm_block_elems": (C.c_int, [C.c_int]),
    "wm_dequant": (C.c_int, [C.c_int, _vp, _i64, _vp, _vp]),
    "wm_quantize": (C.c_int, [C.c_int, _vp, _i64, _vp, _vp]),
    "wm_quantize_host": (C.c_int, [C.c_int, _vp, _i64, _vp]),
    "wm_quant_matvec": (C.c_int, [C.c_int, _vp, _vp, C.c_int, C.c_int, _vp, _vp, _i64, _vp]),
    "wm_router_workspace_size": (_i64, [C.c_int]),
    "wm_router_logits": (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, _vp]),
    "wm_router_topk": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _i64, _vp]),
    "wm_workspace_size": (_i64, [C.POINTER(LayerDesc), C.c_int]),
    "wm_workspace_reset": (C.c_int, [C.POINTER(LayerDesc), C.c_int, _vp, _i64, _vp]),
    "wm_workspace_status": (C.c_int, [_vp, _i64, C.POINTER(C.c_int32)]),
    "wm_workspace_timeline": (C.c_int, [C.POINTER(LayerDesc), C.c_int, C.POINTER(_i64), C.POINTER(_i64)]),
    "wm_device_clock_khz": (_i64, []),
    "wm_workspace_trace": (C.c_int, [C.POINTER(LayerDesc), C.c_int, C.POINTER(_i64), C.POINTER(_i64),
                                     C.POINTER(_i64)]),
    "wm_moe_decode": (C.c_int, [C.POINTER(LayerDesc), _vp, _vp, _vp, _i64, C.c_int, C.c_int, _vp]),
    "wm_moe_decode_forced": (C.c_int, [C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _i64, C.c_int, C.c_int,
                                       _vp]),
    "wm_moe_decode_stack": (C.c_int, [C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, _vp]),
    "wm_noalloc_init": (C.c_int, []),
    "wm_noalloc_scratch_bytes": (_i64, []),
    "wm_moe_decode_noalloc": (C.c_int, [C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp]),
    "wm_noalloc_status": (C.c_int, [C.POINTER(C.c_int32)]),
    "wm_pool_slot_bytes": (_i64, [_i64, _i64, _i64]),
    "wm_pool_create": (C.c_int, [C.c_void_p, _i64, C.c_int, _i64, _i64, _i64, C.POINTER(C.c_void_p)]),
    "wm_pool_destroy": (C.c_int, [C.c_void_p]),
    "wm_pool_layer": (C.c_int, [C.c_void_p, C.c_void_p]),
    "wm_pool_acquire": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int32), C.c_int, C.c_int, C.c_void_p,
                                  C.c_void_p, C.c_void_p, _i64, _i64, _i64, C.c_void_p, C.c_void_p]),
    "wm_pool_acquire_packed": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int32), C.c_int, C.c_int, C.c_void_p,
                                         _i64, C.c_void_p, C.c_void_p]),
    "wm_pool_release": (C.c_int, [C.c_void_p, C.c_void_p]),
    "wm_pool_stats": (C.c_int, [C.c_void_p, C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64)]),
    "wm_prefill_workspace_size": (_i64, [C.POINTER(LayerDesc), C.c_int]),
    "wm_moe_prefill": (C.c_int, [C.POINTER(LayerDesc), _vp, C.c_int, _vp, _vp, _i64, C.c_int, _vp]),
    "wm_moe_prefill_forced": (C.c_int, [C.POINTER(LayerDesc), _vp, C.c_int, _vp, _vp, _vp, _vp, _i64, C.c_int,
                                        _vp]),
    "wm_prefill_workspace_routing": (C.c_int, [C.POINTER(LayerDesc), C.c_int, C.POINTER(_i64), C.POINTER(_i64),
                                               C.POINTER(_i64)]),
    "wm_expert_ffn": (C.c_int, [_vp, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int, C.c_int, _vp, _vp, _i64,
                                _vp]),
    "wm_expert_workspace_size": (_i64, [C.c_int, C.c_int]),
    "wm_profile_enable": (C.c_int, [C.c_int]),
    "wm_profile_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(_i64), C.c_int]),
    "wm_profile_phase_name": (C.c_char_p, [C.c_int]),
    "gpu_init": (C.c_int, []),
    "gpu_shutdown": (None, []),
    "gpu_is_initialized": (C.c_int, []),
    "gpu_vram_used_mb": (C.c_float, []),
    "gpu_upload_router": (C.c_int, [C.c_int, _vp, C.c_int, C.c_int]),
    "gpu_router": (C.c_int, [C.c_int, _vp, C.c_int, _vp, C.c_int]),
    "gpu_cache_expert": (C.c_int, [C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int]),
    "gpu_cache_expert_typed": (C.c_int, [C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                         C.c_int, C.c_int]),
    "gpu_find_cached_expert": (C.c_int, [C.c_int, C.c_int]),
    "gpu_expert_ffn": (C.c_int, [C.c_int, _vp, C.c_int, C.c_int, _vp, _vp, _vp, C.c_int, C.c_int]),
    "gpu_expert_down": (C.c_int, [C.c_int, _vp, C.c_int, _vp, C.c_int]),
    "gpu_expert_ffn_fused": (C.c_int, [C.c_int, _vp, C.c_int, C.c_int, _vp]),
    "gpu_expert_batch_start": (C.c_int, [_vp, C.c_int]),
    "gpu_expert_batch_add": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_float]),
    "gpu_expert_batch_finish": (C.c_int, [_vp, C.c_int]),
    "gpu_expert_cache_count": (C.c_int, []),
    "gpu_set_expert_limit": (None, [C.c_int]),
}

_lib = None


class WinMoEError(RuntimeError):
    """A library call failed; ``rc`` is its return code (WM_ERR or WM_EINVAL,
    None when the library itself could not be loaded)."""

    def __init__(self, msg: str, rc=None):
        super().__init__(msg)
        self.rc = rc


def load():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise WinMoEError(f"{LIB_PATH} is missing: build it with `python -m winmoe_amd.build` "
                              "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc == WM_OK:
        return
    kind = "invalid argument" if rc == WM_EINVAL else "HIP runtime error"
    raise WinMoEError(f"{what or 'winmoe_hip'} failed: {kind} (rc={rc})", rc)
