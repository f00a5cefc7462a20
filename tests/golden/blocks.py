"""Deterministic random GGUF blocks for the oracle and parity tests (test helper).

Scale fields (fp16 d / dmin) are drawn from a finite range so the blocks are
valid; every other byte is uniform random.  ``zero`` forces d or dmin to 0 so
one term of the K-quant dequant formula can be isolated.
"""
from __future__ import annotations

import numpy as np

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 8, 10, 11, 12, 13, 14
BLOCK_BYTES = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
# byte offsets of the fp16 scale fields: (d, dmin or None)
SCALE_FIELDS = {Q8_0: (0, None), Q2_K: (80, 82), Q3_K: (108, None), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208, None)}


def f16_bits(x) -> np.ndarray:
    return np.atleast_1d(np.asarray(x, np.float32)).astype(np.float16).view(np.uint16)


def rand_blocks(qtype: int, n: int, rng: np.random.Generator, lo=1e-4, hi=2e-2, zero=None) -> np.ndarray:
    bs = BLOCK_BYTES[qtype]
    b = rng.integers(0, 256, size=(n, bs), dtype=np.uint8)
    d_off, m_off = SCALE_FIELDS[qtype]
    for off, name in ((d_off, "d"), (m_off, "dmin")):
        if off is None:
            continue
        v = rng.uniform(lo, hi, size=n).astype(np.float32)
        if zero == name:
            v[:] = 0.0
        b[:, off:off + 2] = f16_bits(v).view(np.uint8).reshape(n, 2)
    return b
