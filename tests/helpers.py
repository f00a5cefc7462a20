"""Shared test helpers (not collected)."""
from __future__ import annotations

import numpy as np


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


def bits32(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_bits_nan(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (bits32(a) == bits32(b))))


def ulp_diff(a, b) -> np.ndarray:
    ia = bits32(a).astype(np.int64)
    ib = bits32(b).astype(np.int64)
    ia = np.where(ia >= 0x80000000, 0x80000000 - ia, ia)
    ib = np.where(ib >= 0x80000000, 0x80000000 - ib, ib)
    return np.abs(ia - ib)


def header_functions(path):
    """Function names declared in a C header (declarations ending in ');')."""
    import re
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*([a-z][A-Za-z0-9_]*)\s*\(", txt, flags=re.M)
    return sorted(set(n for n in names if n.startswith(("wm_", "gpu_"))))
