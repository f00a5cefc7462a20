"""Writes tests/golden/ref_vectors.npz from the reference's own kernels.

Run in the dev container, where oracle/_ref/libwmref.so is built from the
reference sources (``make -C oracle``).  The fixture holds inputs and the
reference's outputs only (data), so tests can pin the oracle on hosts where
the reference build is absent.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

from blocks import Q4_K, Q5_K, Q6_K, Q8_0, rand_blocks  # noqa: E402
from oracle import oracle  # noqa: E402

_fp = C.POINTER(C.c_float)


def fptr(a):
    return a.ctypes.data_as(_fp)


def onehot_dots(fn, blocks, value):
    out = np.empty((blocks.shape[0], 256), np.float32)
    for b in range(blocks.shape[0]):
        blk = np.ascontiguousarray(blocks[b])
        for i in range(256):
            x = np.zeros(256, np.float32)
            x[i] = value
            out[b, i] = fn(blk.ctypes.data_as(C.c_void_p), fptr(x))
    return out


def router_case(seed, E, H):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal(H, dtype=np.float32)
    return x, W


def main():
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libwmref.so not built or CPU unsupported")
    out = {}
    # fp16: all 65536 patterns, as float32 bit patterns
    out["fp16_all_bits"] = np.array([R.ref_fp16_to_fp32(h) for h in range(65536)], np.float32).view(np.uint32)
    rng = np.random.default_rng(20261201)
    # Q8_0 dequant rows
    q8 = rand_blocks(Q8_0, 64, rng)
    deq = np.empty((64, 32), np.float32)
    for b in range(64):
        blk = np.ascontiguousarray(q8[b])
        R.ref_q8_dequant_row(blk.ctypes.data_as(C.c_void_p), 32, fptr(deq[b]))
    out["q8_blocks"], out["q8_deq"] = q8, deq
    # Q6_K: one-hot fp32 dots through the scalar reference dot (exact)
    q6 = rand_blocks(Q6_K, 16, rng)
    out["q6_blocks"], out["q6_onehot"] = q6, onehot_dots(R.ref_q6k_dot_block, q6, 1.0)
    # Q4_K / Q5_K: one-hot 127.0 (Q8_K quantises it exactly: d = 1, q = 127)
    for name, qt, fn in (("q4", Q4_K, R.ref_q4k_dot_q8k), ("q5", Q5_K, R.ref_q5k_dot_q8k)):
        bd = rand_blocks(qt, 12, rng, zero="dmin")
        bm = rand_blocks(qt, 12, rng, zero="d")
        out[f"{name}_blocks_d"], out[f"{name}_onehot_d"] = bd, onehot_dots(fn, bd, 127.0)
        out[f"{name}_blocks_m"], out[f"{name}_onehot_m"] = bm, onehot_dots(fn, bm, 127.0)
    # test_q4k.c:21-40 block dotted with ones through the reference ggml-order dot
    kat = np.zeros(144, np.uint8)
    kat[0:2] = np.array([0x00, 0x3C], np.uint8)
    kat[4] = 1
    kat[16:] = 0x0F
    ones = np.ones(256, np.float32)
    out["q4_kat_block"] = kat
    out["q4_kat_dot"] = np.float32(R.ref_q4k_dot_q8k(kat.ctypes.data_as(C.c_void_p), fptr(ones)))
    # Router cases: (seed, E, H, K)
    cases = [(1, 64, 512, 4), (2, 512, 4096, 10), (3, 512, 4096, 3), (4, 64, 2048, 4)]
    for i, (seed, E, H, K) in enumerate(cases):
        x, W = router_case(seed, E, H)
        if i == 0:
            # planted exact three-way tie on the best expert: ids must come out
            # as 0, top, E-1 (equal logits go to the lower index)
            top = int(np.argmax(W.astype(np.float64) @ x.astype(np.float64)))
            W[0] = W[top]
            W[E - 1] = W[top]
        ids = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        R.ref_router_topk(fptr(x), fptr(W), H, E, K, ids.ctypes.data_as(C.POINTER(C.c_int32)), fptr(w))
        out[f"router{i}_case"] = np.array([seed, E, H, K], np.int64)
        out[f"router{i}_ids"], out[f"router{i}_w"] = ids, w
        out[f"router{i}_wsum"] = np.float64(W.astype(np.float64).sum())
        if i == 0:
            out["router0_x"], out["router0_W"] = x, W
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_vectors.npz"))


if __name__ == "__main__":
    main()
