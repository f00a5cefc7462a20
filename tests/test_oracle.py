"""Pins the CPU oracle (oracle/wm_oracle.c) before anything is compared against it.

Sources of truth, in order: the reference's own kernels compiled from source
(oracle/_ref, when present) and the fixture they produced
(tests/golden/ref_vectors.npz); the reference's known answers (test_q4k.c,
test/q6k_parity.cpp); closed forms and brute force.  Q2_K / Q3_K have no
reference code: they are pinned by per-field known-answer blocks built from the
public block layout, and stay "parity unpinned" against the reference.
"""
import ctypes as C
import os

import numpy as np
import pytest
from scipy.special import expit

from golden.blocks import Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, f16_bits, rand_blocks

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (bits(a) == bits(b))))


# ----------------------------------------------------------------- fp16

def test_fp16_exhaustive_vs_numpy(orc):
    got = np.array([orc.fp16_to_fp32(h) for h in range(65536)], np.float32)
    want = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))   # signed zeros, subnormals, inf


def test_fp16_vs_reference(orc):
    got = np.array([orc.fp16_to_fp32(h) for h in range(65536)], np.float32)
    assert np.array_equal(bits(got), GOLD["fp16_all_bits"])   # incl. the reference's NaN canonicalisation


# ----------------------------------------------------------------- Q8_0 / Q6_K / Q4_K / Q5_K vs reference

def test_q8_0_dequant_vs_reference(orc):
    got = orc.dequant(Q8_0, GOLD["q8_blocks"]).reshape(-1, 32)
    assert np.array_equal(bits(got), bits(GOLD["q8_deq"]))


def test_q8_0_dequant_vs_live_reference(orc):
    R = orc.ref()
    if R is None:
        pytest.skip("reference build not available on this host")
    rng = np.random.default_rng(5)
    blocks = rand_blocks(Q8_0, 256, rng, lo=1e-7, hi=6e4)
    got = orc.dequant(Q8_0, blocks)
    want = np.empty(256 * 32, np.float32)
    R.ref_q8_dequant_row(blocks.ctypes.data_as(C.c_void_p), 256 * 32, want.ctypes.data_as(C.POINTER(C.c_float)))
    assert np.array_equal(bits(got), bits(want))


def test_q6k_dequant_vs_reference_onehot(orc):
    # value equality: a one-hot dot returns +0 where the weight is -0
    got = orc.dequant(Q6_K, GOLD["q6_blocks"]).reshape(-1, 256)
    assert np.array_equal(got, GOLD["q6_onehot"])


@pytest.mark.parametrize("name,qt", [("q4", Q4_K), ("q5", Q5_K)])
def test_q4k_q5k_dequant_vs_reference_onehot(orc, name, qt):
    # x = 127 * e_i quantises exactly under Q8_K (d = 1, q = 127), so the
    # reference integer dot returns fl(127 * d*sc*q) for dmin = 0 blocks and
    # -fl(127 * dmin*m) for d = 0 blocks: both terms are pinned bit-for-bit.
    for part in ("d", "m"):
        got = orc.dequant(qt, GOLD[f"{name}_blocks_{part}"]).reshape(-1, 256)
        want = GOLD[f"{name}_onehot_{part}"]
        assert np.array_equal(got * np.float32(127.0), want), part


def test_q4k_known_answer_480(orc):
    # test_q4k.c:21-40: d = 1, dmin = 0, scales[0] = 1, qs = 0x0F.  ggml layout
    # puts the 15s in weights 0..31 only: dot with ones = 480 (the reference's
    # non-ggml float path prints 240, which the build must not follow).
    w = orc.dequant(Q4_K, GOLD["q4_kat_block"])
    assert w[:32].tolist() == [15.0] * 32 and not w[32:].any()
    assert float(w.sum()) == 480.0
    assert float(GOLD["q4_kat_dot"]) == 480.0


def test_q6k_avx2_vs_scalar_relation(orc):
    """test/q6k_parity.cpp:78-135, with random blocks from numpy in place of its generator."""
    R = orc.ref()
    if R is None:
        pytest.skip("reference build not available on this host")
    rng = np.random.default_rng(0xC0FFEE)
    fp = C.POINTER(C.c_float)
    diffs = []
    for dist in range(3):
        blocks = rand_blocks(Q6_K, 300, rng, lo=1e-3, hi=1.1e-2)
        blocks[:, 192:208] = rng.integers(-30, 31, size=(300, 16)).astype(np.int8).view(np.uint8)
        for b in range(300):
            if dist == 0:
                act = rng.normal(0, 0.1, 256)
            elif dist == 1:
                act = rng.normal(0, 3.0, 256)
            else:
                act = rng.uniform(-10, 10, 256)
            act = act.astype(np.float32)
            blk = np.ascontiguousarray(blocks[b])
            s = R.ref_q6k_dot_block(blk.ctypes.data_as(C.c_void_p), act.ctypes.data_as(fp))
            v = R.ref_q6k_dot_block_avx2(blk.ctypes.data_as(C.c_void_p), act.ctypes.data_as(fp))
            diffs.append(float(v) - float(s))
            if b < 20:   # oracle dequant dotted in fp64 agrees with both
                ref64 = float(orc.dequant(Q6_K, blk).astype(np.float64) @ act.astype(np.float64))
                assert abs(ref64 - s) <= 1e-4 * (1 + abs(ref64))
    d = np.array(diffs)
    assert np.abs(d).max() < 1e-3 and np.sqrt((d ** 2).mean()) < 1e-4


# ----------------------------------------------------------------- Q2_K / Q3_K (no reference code)

def q2k_block(scales, qs, d, dmin):
    b = np.zeros(84, np.uint8)
    b[0:16] = scales
    b[16:80] = qs
    b[80:82] = f16_bits(d).view(np.uint8)
    b[82:84] = f16_bits(dmin).view(np.uint8)
    return b


def test_q2k_single_field_positions(orc):
    # A 2-bit field set to 3 in byte qs[32h+l] at bit 2j must land in exactly
    # weight 128h + 32j + l.
    for h in range(2):
        for j in range(4):
            for l in (0, 5, 15, 16, 31):
                qs = np.zeros(64, np.uint8)
                qs[32 * h + l] = 3 << (2 * j)
                w = orc.dequant(Q2_K, q2k_block(np.full(16, 1, np.uint8), qs, 1.0, 0.0))
                nz = np.flatnonzero(w)
                assert nz.tolist() == [128 * h + 32 * j + l] and w[nz[0]] == 3.0


def test_q2k_scale_and_min_maps(orc):
    # Scale byte 8h+2j covers weights 128h+32j+[0,16), byte 8h+2j+1 covers
    # +[16,32); low nibble multiplies d, high nibble multiplies dmin.
    k = np.arange(16, dtype=np.uint8)
    want_idx = np.array([8 * (i // 128) + 2 * ((i % 128) // 32) + ((i % 32) >= 16) for i in range(256)])
    w = orc.dequant(Q2_K, q2k_block(k, np.full(64, 0x55, np.uint8), 1.0, 0.0))      # q = 1 everywhere
    assert np.array_equal(w, want_idx.astype(np.float32))
    w = orc.dequant(Q2_K, q2k_block((k << 4).astype(np.uint8), np.zeros(64, np.uint8), 0.0, 1.0))
    assert np.array_equal(w, -want_idx.astype(np.float32))
    w = orc.dequant(Q2_K, q2k_block(np.full(16, 0x23, np.uint8), np.full(64, 0xFF, np.uint8), 0.5, 0.25))
    assert np.all(w == np.float32(0.5 * 3 * 3 - 0.25 * 2))


def pack_q3_scales(s6):
    """Pack sixteen 6-bit values into the 12 Q3_K scale bytes (inverse of the layout)."""
    s6 = np.asarray(s6, np.uint8)
    out = np.zeros(12, np.uint8)
    for k in range(16):
        lo, hi = s6[k] & 0xF, s6[k] >> 4
        if k < 8:
            out[k] |= lo
        else:
            out[k - 8] |= lo << 4
        out[8 + (k % 4)] |= hi << (2 * (k // 4))
    return out


def q3k_block(hmask, qs, s6, d):
    b = np.zeros(110, np.uint8)
    b[0:32] = hmask
    b[32:96] = qs
    b[96:108] = pack_q3_scales(s6)
    b[108:110] = f16_bits(d).view(np.uint8)
    return b


def test_q3k_single_field_positions(orc):
    ones_scale = np.full(16, 33, np.uint8)           # every scale = +1
    for h in range(2):
        for j in range(4):
            for l in (0, 7, 15, 16, 31):
                qs = np.zeros(64, np.uint8)
                qs[32 * h + l] = 3 << (2 * j)
                w = orc.dequant(Q3_K, q3k_block(np.full(32, 0xFF, np.uint8), qs, ones_scale, 1.0))
                assert np.flatnonzero(w).tolist() == [128 * h + 32 * j + l] and w[128 * h + 32 * j + l] == 3.0
                # the high-mask bit (4h+j) of hmask[l]: clear -> subtract 4 from that weight only
                hm = np.full(32, 0xFF, np.uint8)
                hm[l] &= ~np.uint8(1 << (4 * h + j))
                w2 = orc.dequant(Q3_K, q3k_block(hm, qs, ones_scale, 1.0))
                diff = np.flatnonzero(w2 != w)
                assert diff.tolist() == [128 * h + 32 * j + l] and w2[diff[0]] == -1.0


def test_q3k_scale_map(orc):
    s6 = (np.arange(16) * 4 + 1).astype(np.uint8)     # 1, 5, ..., 61: every bit of the 6-bit field used
    w = orc.dequant(Q3_K, q3k_block(np.full(32, 0xFF, np.uint8), np.full(64, 0x55, np.uint8), s6, 1.0))
    idx = np.array([8 * (i // 128) + 2 * ((i % 128) // 32) + ((i % 32) >= 16) for i in range(256)])
    assert np.array_equal(w, (s6[idx].astype(np.float32) - 32.0))


# ----------------------------------------------------------------- router

def router_inputs(i):
    seed, E, H, K = (int(v) for v in GOLD[f"router{i}_case"])
    if i == 0:
        return GOLD["router0_x"], GOLD["router0_W"], K
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal(H, dtype=np.float32)
    assert W.astype(np.float64).sum() == float(GOLD[f"router{i}_wsum"])   # same inputs as at fixture time
    return x, W, K


@pytest.mark.parametrize("i", [0, 1, 2, 3])
def test_router_vs_reference(orc, i):
    x, W, K = router_inputs(i)
    ids, w, deg = orc.router_topk(x, W, K)
    assert deg == 0
    assert ids.tolist() == GOLD[f"router{i}_ids"].tolist()
    assert np.array_equal(bits(w), bits(GOLD[f"router{i}_w"]))   # same fp32 logits, same expf


def test_router_vs_live_reference_random(orc):
    R = orc.ref()
    if R is None:
        pytest.skip("reference build not available on this host")
    rng = np.random.default_rng(77)
    for trial in range(20):
        E = int(rng.choice([8, 64, 100, 512]))
        H = int(rng.choice([16, 48, 256, 1000, 4096]))    # includes H % 16 != 0 (scalar tail)
        K = int(rng.integers(1, min(E, 16) + 1))
        W = rng.standard_normal((E, H)).astype(np.float32)
        x = rng.standard_normal(H).astype(np.float32)
        ids, w, _ = orc.router_topk(x, W, K)
        rid = np.empty(K, np.int32)
        rw = np.empty(K, np.float32)
        R.ref_router_topk(x.ctypes.data_as(C.POINTER(C.c_float)), W.ctypes.data_as(C.POINTER(C.c_float)),
                          H, E, K, rid.ctypes.data_as(C.POINTER(C.c_int32)), rw.ctypes.data_as(C.POINTER(C.c_float)))
        assert ids.tolist() == rid.tolist() and same_bits(w, rw), (E, H, K)


def test_router_logits_close_to_fp64(orc):
    x, W, K = router_inputs(1)
    got = orc.router_logits(x, W).astype(np.float64)
    exact = W.astype(np.float64) @ x.astype(np.float64)
    assert np.abs(got - exact).max() < 1e-5
    # top-K from exact logits with the tie rule (desc value, asc index) agrees
    order = np.lexsort((np.arange(exact.size), -exact))
    assert order[:K].tolist() == orc.router_topk(x, W, K)[0].tolist()


def test_router_special_cases(orc):
    E, K = 32, 5
    ids, w, deg = orc.topk_softmax(np.zeros(E, np.float32), K)        # all equal: lowest indices
    assert ids.tolist() == list(range(K)) and np.allclose(w, 1.0 / K) and deg == 0
    lg = np.linspace(-1, 1, E).astype(np.float32)
    lg[E - 1] = np.nan                                                 # NaN is never selected
    ids, w, deg = orc.topk_softmax(lg, K)
    assert ids.tolist() == [E - 2, E - 3, E - 4, E - 5, E - 6]
    assert abs(float(w.sum()) - 1.0) < 1e-6 and np.all(np.diff(w) <= 0)
    ids, w, deg = orc.topk_softmax(np.full(E, -np.inf, np.float32), 2)  # degenerate: index 0 re-picked
    assert deg == 1 and ids.tolist() == [0, 0]
    perm = np.random.default_rng(3).permutation(E).astype(np.float32)
    ids, _, _ = orc.topk_softmax(perm, E)                              # K = E is a full sort
    assert sorted(ids.tolist()) == list(range(E)) and np.all(np.diff(perm[ids]) < 0)


# ----------------------------------------------------------------- expert FFN / MoE layer

def dense(orc, qt, blocks, rows, cols):
    return orc.dequant(qt, blocks).astype(np.float64).reshape(rows, cols)


@pytest.mark.parametrize("types", [(Q8_0, Q8_0, Q8_0), (Q4_K, Q4_K, Q6_K), (Q2_K, Q2_K, Q3_K), (Q5_K, Q4_K, Q8_0)])
def test_expert_ffn_brute_force(orc, types):
    H, I = 512, 256
    gt, ut, dt = types
    rng = np.random.default_rng(11)
    nb = lambda qt, rows, cols: rows * cols // (32 if qt == Q8_0 else 256)
    g = rand_blocks(gt, nb(gt, I, H), rng)
    u = rand_blocks(ut, nb(ut, I, H), rng)
    d = rand_blocks(dt, nb(dt, H, I), rng)
    x = rng.standard_normal(H)
    y, act = orc.expert_ffn(g, gt, u, ut, d, dt, x, H, I, want_act=True)
    gv = dense(orc, gt, g, I, H) @ x
    uv = dense(orc, ut, u, I, H) @ x
    a = gv * expit(gv) * uv
    yv = dense(orc, dt, d, H, I) @ a
    assert np.allclose(act, a, rtol=1e-12, atol=1e-12 * np.abs(a).max())
    assert np.linalg.norm(y - yv) <= 1e-12 * np.linalg.norm(yv)


def tiny_layer(orc, rng, with_shared=True):
    H, I, E, K = 256, 256, 6, 2
    nbg = I * H // 32
    gate = rand_blocks(Q8_0, E * nbg, rng)
    up = rand_blocks(Q8_0, E * nbg, rng)
    down = rand_blocks(Q8_0, E * nbg, rng)
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    shared = sh_inp = None
    if with_shared:
        shared = (rand_blocks(Q8_0, nbg, rng), rand_blocks(Q8_0, nbg, rng), rand_blocks(Q8_0, nbg, rng))
        sh_inp = (rng.standard_normal(H) * 0.02).astype(np.float32)
    L = orc.make_layer(H, I, E, K, (Q8_0, Q8_0, Q8_0), router=router, gate=gate, up=up, down=down,
                       shared=shared, sh_types=(Q8_0, Q8_0, Q8_0) if with_shared else None, sh_gate_inp=sh_inp)
    return L, dict(gate=gate, up=up, down=down, router=router, shared=shared, sh_inp=sh_inp, H=H, I=I, E=E, K=K)


def test_moe_layer_vs_dense(orc):
    rng = np.random.default_rng(21)
    L, p = tiny_layer(orc, rng)
    x = rng.standard_normal(p["H"]).astype(np.float32)
    ids, w, out, rc = orc.moe_layer(L, x)
    H, I, E, K = p["H"], p["I"], p["E"], p["K"]
    logits = p["router"].astype(np.float64) @ x.astype(np.float64)
    order = np.lexsort((np.arange(E), -logits))[:K]
    assert ids.tolist() == order.tolist()
    sel = logits[order]
    wv = np.exp(sel - sel.max())
    wv /= wv.sum()
    assert np.allclose(w, wv, rtol=1e-6)
    per = I * H // 32 * 34
    acc = np.zeros(H)
    xd = x.astype(np.float64)
    for k, e in enumerate(order):
        sl = slice(e * per, (e + 1) * per)
        gv = dense(orc, Q8_0, p["gate"][e * (per // 34):(e + 1) * (per // 34)], I, H) @ xd
        uv = dense(orc, Q8_0, p["up"][e * (per // 34):(e + 1) * (per // 34)], I, H) @ xd
        yv = dense(orc, Q8_0, p["down"][e * (per // 34):(e + 1) * (per // 34)], H, I) @ (gv * expit(gv) * uv)
        acc += float(w[k]) * yv
        del sl
    sg, su, sd = p["shared"]
    gv = dense(orc, Q8_0, sg, I, H) @ xd
    uv = dense(orc, Q8_0, su, I, H) @ xd
    ys = dense(orc, Q8_0, sd, H, I) @ (gv * expit(gv) * uv)
    acc += expit(float(p["sh_inp"].astype(np.float64) @ xd)) * ys
    assert np.linalg.norm(out - acc) <= 1e-12 * np.linalg.norm(acc)


def test_moe_layer_vs_reference_cpu_path(orc):
    """Same routing bit-for-bit; outputs agree to the reference's int8-activation error."""
    if orc.ref() is None:
        pytest.skip("reference build not available on this host")
    rng = np.random.default_rng(31)
    L, p = tiny_layer(orc, rng)
    x = rng.standard_normal(p["H"]).astype(np.float32)
    ids, w, out, _ = orc.moe_layer(L, x)
    rids, rw, rout, port = orc.ref_moe_layer_cpu(L, x)
    assert port == 0
    assert ids.tolist() == rids.tolist() and same_bits(w, rw)
    rel = np.linalg.norm(rout - out) / np.linalg.norm(out)
    assert rel < 3e-2, rel      # Q8_K activation quantisation in the reference path (~7e-3 typical)


# ------------------------------------------------------------------ RMSNorm (the step's producer)

def test_rmsnorm_vs_live_reference(orc):
    """wmo_rmsnorm == the reference's rmsnorm (attention.h:29-44, compiled from
    source), bit for bit, including dims with a scalar tail."""
    R = orc.ref()
    if R is None:
        pytest.skip("reference build not available on this host")
    rng = np.random.default_rng(5)
    fp = C.POINTER(C.c_float)
    for dim in (8, 13, 256, 1000, 2048, 4096):
        for scale in (1e-3, 1.0, 30.0):
            x = (rng.standard_normal(dim) * scale).astype(np.float32)
            w = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
            got = orc.rmsnorm(x, w)
            ref = np.empty(dim, np.float32)
            R.wmref_rmsnorm(ref.ctypes.data_as(fp), x.ctypes.data_as(fp), w.ctypes.data_as(fp), dim)
            assert same_bits(got, ref), (dim, scale)


def test_rmsnorm_closed_forms(orc):
    """Rows whose fp64 sum of squares is exact: a constant row (ss = dim c^2)
    and a one-hot row (ss = v^2), with the float scale formed as written."""
    dim = 4096
    w = np.linspace(0.5, 1.5, dim, dtype=np.float32)
    for c in (0.5, 3.0, -2.0):
        x = np.full(dim, c, np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(np.float64(dim) * c * c / dim) + np.float32(1e-6))
        assert same_bits(orc.rmsnorm(x, w), (x * scale) * w)
    x = np.zeros(dim, np.float32)
    x[17] = 8.0
    scale = np.float32(1.0) / np.sqrt(np.float32(64.0 / dim) + np.float32(1e-6))
    assert same_bits(orc.rmsnorm(x, w), (x * scale) * w)


@pytest.mark.parametrize("qt", [Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K])
def test_dequant_block_sums(orc, qt):
    """The per-block checksums the full-trace dequant test compares: each
    block's sums of its dequantised bit patterns (plain and position-weighted),
    here computed again in numpy from wmo_dequant; threaded splits agree with
    one call; a change to one weight of one block moves that block's sums
    and no other's."""
    rng = np.random.default_rng(qt)
    n = 257
    b = rand_blocks(qt, n, rng)
    ne = {Q8_0: 32}.get(qt, 256)
    u = orc.dequant(qt, b).view(np.uint32).astype(np.int64).reshape(n, ne)
    s1, s2 = orc.dequant_block_sums(qt, b)
    assert np.array_equal(s1, u.sum(1))
    assert np.array_equal(s2, (u * np.arange(1, ne + 1)).sum(1))
    t1, t2 = orc.dequant_block_sums(qt, b, threads=5)
    assert np.array_equal(s1, t1) and np.array_equal(s2, t2)
    b2 = b.copy()
    b2[100, -1] ^= 0x11          # the last quant byte of block 100
    c1, c2 = orc.dequant_block_sums(qt, b2)
    moved = (c1 != s1) | (c2 != s2)
    assert moved[100] and moved.sum() == 1
