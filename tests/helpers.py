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


# ------------------------------------------------------------ RMSNorm sum orders

def rms_ss_kernel_order(h) -> float:
    """Sum of squares of h (fp32) in the persistent decode step's order: lane
    l of 64 keeps four fp64 sums s_c over i = 4l + 256k + c (k in order),
    ss_l = (s_0 + s_1) + (s_2 + s_3), then an xor butterfly over the lanes
    (32, 16, ..., 1)."""
    v = np.asarray(h, np.float32).astype(np.float64)
    H = v.size
    lanes = np.zeros(64)
    for l in range(64):
        s = [0.0, 0.0, 0.0, 0.0]
        if 4 * l < H:
            for k in range((H + 255) // 256):
                for c in range(4):
                    i = 4 * l + 256 * k + c
                    if i < H:
                        s[c] += v[i] * v[i]
        lanes[l] = (s[0] + s[1]) + (s[2] + s[3])
    for m in (32, 16, 8, 4, 2, 1):
        lanes = lanes + lanes[np.arange(64) ^ m]
    return float(lanes[0])


def rms_ss_index_order(h) -> float:
    """attention.h:31-33: ss += (double)x[i] * x[i] for i in index order."""
    ss = 0.0
    for x in np.asarray(h, np.float32).astype(np.float64):
        ss += x * x
    return ss


def rms_scale(ss: float, H: int, eps: float = 1e-6):
    """scale = 1 / sqrtf((float)(ss / H) + eps), all in fp32 after the cast."""
    return np.float32(1.0) / np.sqrt(np.float32(ss / H) + np.float32(eps), dtype=np.float32)


def rms_boundary_vector(H: int) -> np.ndarray:
    """h[0] = 4097, every other element 2^-16: 4097^2 = 16785409 needs 25
    significant bits, so ss / H (H a power of two) sits exactly on a float
    rounding boundary in index order (each 2^-32 square is below half an ulp
    of the running sum and is lost), while any order that adds the small
    squares among themselves first ends above it: the two orders round
    (float)(ss / H) differently."""
    h = np.full(H, 2.0 ** -16, np.float32)
    h[0] = 4097.0
    return h
