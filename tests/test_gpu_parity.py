"""GPU parity: the HIP path through the C-ABI vs the CPU oracle on the same bytes.

Bars: dequantised weights and router logits bit-exact, top-K ids exact,
routing weights within 2 ulp (device expf), expert / layer outputs rel-L2
<= 1e-3 against the oracle's fp32-dequant + fp64 maths.
"""
import numpy as np
import pytest

from golden.blocks import Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, rand_blocks
from helpers import (rel_l2, rms_boundary_vector, rms_ss_index_order, rms_ss_kernel_order, same_bits_nan,
                     ulp_diff)

pytestmark = pytest.mark.gpu

TYPES = [Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]
LAYER_TOL = 1e-3          # rel-L2 of layer / expert outputs vs the fp64 oracle
MATVEC_TOL = 2e-4         # rel-L2 of a single quantised matrix-vector product


@pytest.fixture(scope="module")
def wm():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import winmoe_amd
    winmoe_amd.load()
    return winmoe_amd


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def case(msg):
    print(f"[case] {msg}", flush=True)


# ------------------------------------------------------------------ dequant / quantise

@pytest.mark.parametrize("t", TYPES)
def test_dequant_bit_exact(wm, orc, t):
    rng = np.random.default_rng(100 + t)
    for nb in (1, 3, 16, 17, 129, 1000):
        case(f"dequant type={t} nblocks={nb}")
        blocks = rand_blocks(t, nb, rng, lo=1e-6, hi=30.0)
        got = host(wm.dequantize(dev(blocks.reshape(-1)), t))
        assert same_bits_nan(got, orc.dequant(t, blocks)), (t, nb)


@pytest.mark.parametrize("t", TYPES)
def test_dequant_special_scales(wm, orc, t):
    from golden.blocks import SCALE_FIELDS
    rng = np.random.default_rng(7 + t)
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x3C00],
                        np.uint16)
    blocks = rand_blocks(t, len(specials) * 2, rng)
    d_off, m_off = SCALE_FIELDS[t]
    for i, s in enumerate(specials):
        blocks[i, d_off:d_off + 2] = np.array([s], np.uint16).view(np.uint8)
        if m_off is not None:
            blocks[len(specials) + i, m_off:m_off + 2] = np.array([s], np.uint16).view(np.uint8)
    case(f"dequant special fp16 scales type={t}")
    got = host(wm.dequantize(dev(blocks.reshape(-1)), t))
    assert same_bits_nan(got, orc.dequant(t, blocks))


def test_dequant_rejects_misaligned(wm):
    import torch
    buf = torch.zeros(34 * 8, dtype=torch.uint8, device="cuda")
    with pytest.raises(wm.WinMoEError):
        wm.dequantize(buf[34:34 * 4], Q8_0)        # 34-byte offset: 2-byte aligned only


@pytest.mark.parametrize("t", TYPES)
def test_quantize_device_matches_host(wm, t):
    import ctypes as C
    rng = np.random.default_rng(t)
    x = (rng.standard_normal(256 * 300) * 0.02).astype(np.float32)
    x[:256] *= 1e-30      # tiny values, subnormal fp16 scales
    x[256:512] = 0.0
    case(f"quantize type={t}")
    got = host(wm.quantize(dev(x), t))
    ref = np.zeros_like(got)
    assert wm.load().wm_quantize_host(t, x.ctypes.data, x.size, ref.ctypes.data) == 0
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ router

def router_case(E, H, seed, tie=False, nan_row=None):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal(H, dtype=np.float32)
    if tie:
        top = int(np.argmax(W.astype(np.float64) @ x.astype(np.float64)))
        W[0] = W[top]
        W[E - 1] = W[top]
    if nan_row is not None:
        W[nan_row, 5] = np.nan
    return x, W


@pytest.mark.parametrize("E,H,K,seed,tie", [(512, 4096, 10, 1, False), (512, 4096, 3, 2, True),
                                            (64, 2048, 4, 3, False), (64, 512, 4, 4, True),
                                            (100, 1000, 7, 5, False), (1024, 256, 16, 6, True)])
def test_router_bit_exact(wm, orc, E, H, K, seed, tie):
    x, W = router_case(E, H, seed, tie=tie, nan_row=E // 3)
    case(f"router E={E} H={H} K={K}")
    lg = host(wm.router_logits(dev(x), dev(W)))
    assert same_bits_nan(lg, orc.router_logits(x, W))
    ids, w = wm.router_topk(dev(x), dev(W), K)
    oid, ow, _ = orc.router_topk(x, W, K)
    assert host(ids).tolist() == oid.tolist()
    assert ulp_diff(host(w), ow).max() <= 2
    if tie:
        assert host(ids)[:3].tolist()[0] == 0


# ------------------------------------------------------------------ matvec / expert

@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("inp", [256, 512, 1024, 2048, 4096])
def test_quant_matvec(wm, orc, t, inp):
    rng = np.random.default_rng(inp + t)
    rows = 96
    nb = rows * inp // orc.BLOCK_ELEMS[t]
    W = rand_blocks(t, nb, rng)
    x = rng.standard_normal(inp).astype(np.float32)
    case(f"matvec type={t} in={inp}")
    y = host(wm.quant_matvec(dev(W.reshape(-1)), dev(x), rows, inp, t))
    want = orc.matvec(t, W, x, rows, inp)
    assert rel_l2(y, want) <= MATVEC_TOL


@pytest.mark.parametrize("types", [(Q8_0, Q8_0, Q8_0), (Q4_K, Q4_K, Q6_K), (Q2_K, Q2_K, Q3_K), (Q5_K, Q5_K, Q5_K),
                                   (Q4_K, Q8_0, Q2_K)])
def test_expert_ffn(wm, orc, types):
    import torch
    H, I = 4096, 1024
    g = torch.Generator(device="cuda").manual_seed(5)
    gt, ut, dt = types
    mats = []
    for t, r, c in ((gt, I, H), (ut, I, H), (dt, H, I)):
        w = torch.randn(r * c, generator=g, device="cuda") * 0.02
        mats.append(wm.quantize(w, t))
    x = torch.randn(H, generator=g, device="cuda")
    case(f"expert_ffn types={types}")
    y = host(wm.expert_ffn(*mats, x, H, I, types))
    want = orc.expert_ffn(host(mats[0]), gt, host(mats[1]), ut, host(mats[2]), dt, host(x), H, I)
    assert rel_l2(y, want) <= LAYER_TOL


# ------------------------------------------------------------------ MoE layer

def oracle_token(orc, sl, x, ids=None, w=None):
    """fp64 MoE block for one token over the synthetic layer's bytes."""
    from winmoe_amd.moe import matrix_bytes
    cfg, L = sl.cfg, sl.layer
    H, I, K = cfg.H, cfg.I, cfg.K
    if ids is None:
        ids, w, _ = orc.router_topk(x, host(sl.router), K)
    gt, ut, dt = cfg.types
    pg, pu, pd = matrix_bytes(gt, I, H), matrix_bytes(ut, I, H), matrix_bytes(dt, H, I)
    out = np.zeros(H)
    for k, e in enumerate(ids):
        e = int(e)
        y = orc.expert_ffn(host(sl.gate[e * pg:(e + 1) * pg]), gt, host(sl.up[e * pu:(e + 1) * pu]), ut,
                           host(sl.down[e * pd:(e + 1) * pd]), dt, x, H, I)
        out += float(w[k]) * y
    if sl.shared is not None:
        s = sl.shared
        Is = s.inter or I
        ys = orc.expert_ffn(host(s.gate), s.types[0], host(s.up), s.types[1], host(s.down), s.types[2], x, H, Is)
        gate = 1.0
        if s.gate_inp is not None:
            gate = orc.lib().wmo_sigmoid(float(host(s.gate_inp).astype(np.float64) @ x.astype(np.float64)))
        out += gate * ys
    return np.asarray(ids), np.asarray(w), out


def decode_check(wm, orc, cfg, E, tokens, seed_offset=0):
    from winmoe_amd import synth
    sl = synth.build_layer(cfg, E=E, max_tokens=max(tokens, 4))
    X = synth.make_hidden(cfg, tokens=tokens, seed_offset=seed_offset)
    for t in range(tokens):
        case(f"decode {cfg.name} E={E} token={t}")
        out = host(sl.layer.decode(X[t]))
        ids_t, w_t = sl.layer.trace()
        xi = host(X[t])
        oid, ow, ref = oracle_token(orc, sl, xi)
        assert host(ids_t[t]).tolist() == oid.tolist(), t
        assert ulp_diff(host(w_t[t]), ow).max() <= 2
        assert rel_l2(out, ref) <= LAYER_TOL, (t, rel_l2(out, ref))
    assert sl.layer.status() == 0
    return sl


def test_decode_c1_full(wm, orc):
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c1"]
    decode_check(wm, orc, cfg, E=cfg.E, tokens=3)


def test_decode_c2_shape_small_e(wm, orc):
    from winmoe_amd import synth
    decode_check(wm, orc, synth.CONFIGS["c2"], E=24, tokens=3)


def test_decode_c2_full(wm, orc):
    from winmoe_amd import synth
    sl = decode_check(wm, orc, synth.CONFIGS["c2"], E=512, tokens=2)
    hits = host(sl.layer.hits())
    assert hits.sum() == 2 * 10


def test_decode_c3_types(wm, orc):
    from winmoe_amd import synth
    decode_check(wm, orc, synth.CONFIGS["c3"], E=16, tokens=3)


def test_decode_forced_c4_types(wm, orc):
    import torch
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c4"]
    E, T = 24, 4
    sl = synth.build_layer(cfg, E=E, max_tokens=8)
    X = synth.make_hidden(cfg, tokens=T)
    ids, w = synth.forced_routes(cfg, E=E, tokens=T)
    for t in range(T):
        case(f"forced decode {cfg.name} token={t}")
        out = host(sl.layer.decode_forced(X[t], dev(ids[t]), dev(w[t])))
        _, _, ref = oracle_token(orc, sl, host(X[t]), ids[t], w[t])
        assert rel_l2(out, ref) <= LAYER_TOL
    tid, tw = sl.layer.trace()
    assert np.array_equal(host(tid[:T]), ids) and np.array_equal(host(tw[:T]), w)
    assert sl.layer.status() == 0
    del torch


def test_forced_bad_expert_id_flags_and_zeroes(wm, orc):
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c1"]
    sl = synth.build_layer(cfg, E=8, max_tokens=4)
    x = synth.make_hidden(cfg, tokens=1)[0]
    ids = np.array([1, 99, 2, -1], np.int32)
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    case("forced decode with out-of-range ids")
    out = host(sl.layer.decode_forced(x, dev(ids), dev(w)))
    assert sl.layer.status() & wm._lib.STATUS_BAD_EXPERT_ID
    _, _, ref = oracle_token(orc, sl, host(x), np.array([1, 2]), np.array([0.4, 0.2]))
    assert rel_l2(out, ref) <= LAYER_TOL


def test_decode_deterministic(wm):
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c2"]
    sl = synth.build_layer(cfg, E=16, max_tokens=4)
    x = synth.make_hidden(cfg, tokens=1)[0]
    case("decode determinism")
    a = host(sl.layer.decode(x))
    b = host(sl.layer.decode(x))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------------ gpu_offload.h shims

def test_legacy_expert_cache_and_ffn(wm, orc):
    import ctypes as C
    import torch
    L = wm.load()
    H, I = 4096, 1024
    g = torch.Generator(device="cuda").manual_seed(9)
    mats = [host(wm.quantize(torch.randn(r * c, generator=g, device="cuda") * 0.02, t))
            for t, r, c in ((Q4_K, I, H), (Q4_K, I, H), (Q5_K, H, I))]
    x = np.random.default_rng(0).standard_normal(H).astype(np.float32)
    case("legacy gpu_* shims")
    assert L.gpu_init() == 0 and L.gpu_is_initialized() == 1
    slot = L.gpu_cache_expert(3, 213, mats[0].ctypes.data, mats[0].size, mats[1].ctypes.data, mats[1].size,
                              mats[2].ctypes.data, mats[2].size)
    assert slot >= 0 and L.gpu_find_cached_expert(3, 213) == slot and L.gpu_find_cached_expert(3, 212) == -1
    out = np.zeros(H, np.float32)
    assert L.gpu_expert_ffn_fused(slot, x.ctypes.data, H, I, out.ctypes.data) == 0
    want = orc.expert_ffn(mats[0], Q4_K, mats[1], Q4_K, mats[2], Q5_K, x, H, I)
    assert rel_l2(out, want) <= LAYER_TOL
    go, uo, eo = np.zeros(I, np.float32), np.zeros(I, np.float32), np.zeros(H, np.float32)
    assert L.gpu_expert_ffn(slot, x.ctypes.data, H, I, go.ctypes.data, uo.ctypes.data, eo.ctypes.data, 12, 13) == 0
    assert rel_l2(go, orc.matvec(Q4_K, mats[0], x, I, H)) <= MATVEC_TOL
    # batch API: two weighted copies of the same expert
    acc = np.zeros(H, np.float32)
    assert L.gpu_expert_batch_start(x.ctypes.data, H) == 0
    assert L.gpu_expert_batch_add(slot, H, I, C.c_float(0.25)) == 0
    assert L.gpu_expert_batch_add(slot, H, I, C.c_float(0.5)) == 0
    assert L.gpu_expert_batch_finish(acc.ctypes.data, H) == 0
    assert rel_l2(acc, 0.75 * want) <= LAYER_TOL
    # router shim
    E = 64
    W = (np.random.default_rng(1).standard_normal((E, H)) * 0.02).astype(np.float32)
    lg = np.zeros(E, np.float32)
    assert L.gpu_upload_router(0, W.ctypes.data, H, E) == 0
    assert L.gpu_router(0, x.ctypes.data, H, lg.ctypes.data, E) == 0
    assert same_bits_nan(lg, orc.router_logits(x, W))
    assert L.gpu_expert_cache_count() == 1 and L.gpu_vram_used_mb() > 0
    L.gpu_shutdown()
    assert L.gpu_is_initialized() == 0


# ------------------------------------------------------------------ fused step vs per-phase launches

_KERNEL_FLAGS = {"persist": 8, "item": 4}


@pytest.mark.parametrize("kernel", ["persist", "item"])
@pytest.mark.parametrize("name,E,tokens", [("c1", 64, 4), ("c1", 1000, 3), ("c1", 700, 3), ("c2", 40, 6),
                                           ("c2", 512, 3), ("c3", 24, 4), ("c4", 24, 4)])
def test_fused_step_matches_multi_kernel(wm, name, E, tokens, kernel):
    """One fused launch per token (persistent or work-item-list kernel) == the
    per-phase kernel sequence, bit for bit, over several consecutive tokens
    (the counters and hand-off tags carry over between launches).  E=512 puts
    two router rows on each workgroup of the persistent kernel, E=1000 four
    (the last workgroups have fewer or none), E=700 three."""
    from winmoe_amd import synth
    cfg = synth.CONFIGS[name]
    sl = synth.build_layer(cfg, E=E, max_tokens=8)
    fused = synth.twin_layer(sl, multi_kernel=False, flags=_KERNEL_FLAGS[kernel])
    multi = synth.twin_layer(sl, multi_kernel=True)
    X = synth.make_hidden(cfg, tokens=tokens)
    routes = synth.forced_routes(cfg, E=E, tokens=tokens) if cfg.routing != "router" else None
    for t in range(tokens):
        case(f"{kernel} vs multi {name} E={E} token={t}")
        if routes is None:
            a = host(fused.decode(X[t]))
            b = host(multi.decode(X[t]))
        else:
            ids, w = dev(routes[0][t]), dev(routes[1][t])
            a = host(fused.decode_forced(X[t], ids, w))
            b = host(multi.decode_forced(X[t], ids, w))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
    ta, wa = fused.trace()
    tb, wb = multi.trace()
    assert np.array_equal(host(ta[:tokens]), host(tb[:tokens]))
    assert np.array_equal(host(wa[:tokens]).view(np.uint32), host(wb[:tokens]).view(np.uint32))
    assert np.array_equal(host(fused.hits()), host(multi.hits()))
    assert fused.status() == 0 and multi.status() == 0



@pytest.mark.parametrize("H,I,K,shared", [(256, 64, 2, True), (512, 128, 3, False), (1024, 256, 4, True),
                                          (4096, 64, 8, True), (2048, 128, 10, False)])
def test_decode_narrow_intermediate(wm, orc, H, I, K, shared):
    """Narrow intermediate widths: a slot's SwiGLU hand-off (two outputs per
    tagged word) is one act tile of 256 or 512 bytes, less than one DMA
    kilobyte; with 8 slots or more the act tiles hold 16 segments.  Decode
    against the oracle, the fused step against the per-phase kernels bit for
    bit, and a decode with a fused RMSNorm (which only the persistent kernel
    runs) against the plain decode of the normalised input."""
    import torch
    from winmoe_amd import synth
    from winmoe_amd.moe import MoELayer
    E = 32
    cfg = synth.LayerConfig(f"narrow_h{H}_i{I}_k{K}", E=E, K=K, H=H, I=I, types=(Q8_0, Q8_0, Q8_0),
                            shared_types=(Q8_0, Q8_0, Q8_0) if shared else None, shared_inter=I if shared else 0,
                            shared_gate_inp=shared, tokens=1, seed=11)
    sl = decode_check(wm, orc, cfg, E=E, tokens=3)
    fused = synth.twin_layer(sl, multi_kernel=False, flags=_KERNEL_FLAGS["persist"])
    multi = synth.twin_layer(sl, multi_kernel=True)
    X = synth.make_hidden(cfg, tokens=3, seed_offset=5)
    for t in range(3):
        case(f"narrow H={H} I={I} K={K} fused vs multi token={t}")
        a = host(fused.decode(X[t]))
        b = host(multi.decode(X[t]))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
    g = torch.Generator(device="cuda").manual_seed(3)
    w = (1.0 + 0.1 * torch.randn(H, generator=g, device="cuda")).float()
    normed = MoELayer(H, I, E, K, sl.router, sl.gate, sl.up, sl.down, cfg.types, shared=sl.shared, max_tokens=4,
                      norm_w=w, add_residual=False)
    h = (3.0 * torch.randn(H, generator=g, device="cuda")).contiguous()
    hh = host(h)
    case(f"narrow H={H} I={I} K={K} rmsnorm")
    got = host(normed.decode(h))
    want = host(fused.decode(dev(orc.rmsnorm(hh, host(w)))))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert normed.status() == 0 and fused.status() == 0 and multi.status() == 0


@pytest.mark.parametrize("E,K", [(64, 4), (512, 10), (1000, 16)])
def test_decode_routing_ties_and_nan_row(wm, orc, E, K):
    """The persistent step's routing with planted ties (rows 0 and E-1 copy
    the token's top row: equal logits go to the smaller index first) and a
    router row holding a NaN (never picked), at one key per lane (E=64),
    eight (E=512) and sixteen (E=1000): ids as the oracle's K-pass arg-max,
    weights within 2 ulp, output bit for bit as the per-phase kernels'."""
    import torch
    from winmoe_amd import synth
    cfg = synth.LayerConfig(f"ties_e{E}_k{K}", E=E, K=K, H=1024, I=256, types=(Q8_0, Q8_0, Q8_0),
                            shared_types=(Q8_0, Q8_0, Q8_0), shared_inter=256, shared_gate_inp=True, tokens=1,
                            seed=21)
    sl = synth.build_layer(cfg, E=E, max_tokens=4)
    X = synth.make_hidden(cfg, tokens=2, seed_offset=9)
    xh = host(X[0])
    W = host(sl.router).copy()
    top = int(np.argmax(W.astype(np.float64) @ xh.astype(np.float64)))
    W[0] = W[top]
    W[E - 1] = W[top]
    W[E // 3, 7] = np.nan
    sl.router.copy_(torch.from_numpy(W).to(sl.router.device))
    multi = synth.twin_layer(sl, multi_kernel=True)
    for t in range(2):
        case(f"ties E={E} K={K} token={t}")
        out = host(sl.layer.decode(X[t]))
        ids_t, w_t = sl.layer.trace()
        oid, ow, ref = oracle_token(orc, sl, host(X[t]))
        assert host(ids_t[t]).tolist() == oid.tolist(), t
        assert E // 3 not in oid.tolist()
        assert ulp_diff(host(w_t[t]), ow).max() <= 2
        assert rel_l2(out, ref) <= LAYER_TOL
        assert np.array_equal(out.view(np.uint32), host(multi.decode(X[t])).view(np.uint32)), t
    tied = sorted({0, top, E - 1})
    assert host(sl.layer.trace()[0][0])[:len(tied)].tolist() == tied
    assert sl.layer.status() == 0 and multi.status() == 0

# ------------------------------------------------------------------ prefill

def _pf_cfg(E, K, H, I, shared=False, routing="router"):
    from winmoe_amd import synth
    return synth.LayerConfig(f"pf_e{E}_k{K}_h{H}_i{I}", E=E, K=K, H=H, I=I, types=(Q8_0, Q8_0, Q8_0),
                             shared_types=(Q8_0, Q8_0, Q8_0) if shared else None, shared_inter=I if shared else 0,
                             shared_gate_inp=shared, tokens=1, routing=routing, x_dtype="bf16", seed=3)


@pytest.mark.parametrize("shared", [False, True])
def test_prefill_router_matches_oracle(wm, orc, shared):
    """Batched prefill routed by the router == the oracle token by token: ids
    exact, weights within 2 ulp, outputs within the layer bar."""
    from winmoe_amd import synth
    cfg = _pf_cfg(E=48, K=4, H=1024, I=512, shared=shared)
    T = 40
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg, tokens=T)
    case(f"prefill router shared={shared} T={T}")
    out = host(sl.layer.prefill(X))
    ids, w = (host(a) for a in sl.layer.prefill_routing(T))
    for t in range(T):
        oid, ow, ref = oracle_token(orc, sl, host(X[t].float()))
        assert ids[t].tolist() == oid.tolist(), t
        assert ulp_diff(w[t], ow).max() <= 2, t
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    assert sl.layer.prefill_status() == 0


def test_prefill_router_kernels_agree(wm):
    """The two prefill router kernels (16-byte aligned router rows and H a
    multiple of 128: the vectorised tiles; otherwise the plain ones) give the
    same logits, so the same routing and outputs bit for bit: the same layer
    run with its router at a 16-byte aligned address and at one 4 bytes past
    it (E = 40, H = 1024, 37 tokens: partial tiles both ways)."""
    import torch
    from winmoe_amd import synth
    from winmoe_amd.moe import MoELayer
    cfg = _pf_cfg(E=40, K=4, H=1024, I=512)
    T = 37
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg, tokens=T)
    E, H = cfg.E, cfg.H
    buf = torch.zeros(E * H + 4, dtype=torch.float32, device="cuda")
    shifted = buf[1:1 + E * H].view(E, H)
    shifted.copy_(sl.router)
    assert shifted.data_ptr() % 16 == 4 and sl.router.data_ptr() % 16 == 0
    L = sl.layer
    moved = MoELayer(H, cfg.I, E, cfg.K, shifted, L.gate_exps, L.up_exps, L.down_exps, L.types, max_tokens=T)
    case(f"prefill router kernels T={T}")
    a = host(L.prefill(X))
    b = host(moved.prefill(X))
    ia, wa = (host(v) for v in L.prefill_routing(T))
    ib, wb = (host(v) for v in moved.prefill_routing(T))
    assert np.array_equal(ia, ib)
    assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert L.prefill_status() == 0 and moved.prefill_status() == 0


def test_prefill_scales_and_narrow_shared(wm, orc):
    """Tokens whose magnitudes span 1e-6 .. 1e4 (one all zero, one with a
    single huge entry), a shared expert half as wide as the routed ones, an
    odd token count; forced routing."""
    import torch
    from winmoe_amd import synth
    cfg = synth.LayerConfig("pf_e24_k3_h1024_i512_s256", E=24, K=3, H=1024, I=512, types=(Q8_0, Q8_0, Q8_0),
                            shared_types=(Q8_0, Q8_0, Q8_0), shared_inter=256, shared_gate_inp=True, tokens=1,
                            routing="zipf", x_dtype="bf16", seed=11)
    T = 37
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg, tokens=T).float()
    scale = torch.logspace(-6, 4, T, device=X.device)
    X = X * scale[:, None]
    X[5] = 0.0
    X[9, 100] = 3.0e4
    X = X.to(torch.bfloat16)
    rng = np.random.default_rng(7)
    ids = np.stack([rng.choice(24, 3, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, 3)).astype(np.float32)
    case(f"prefill scales T={T}")
    out = host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    for t in range(T):
        _, _, ref = oracle_token(orc, sl, host(X[t].float()), ids=ids[t], w=w[t])
        if t == 5:
            assert np.abs(out[t]).max() == 0.0
            continue
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    assert sl.layer.prefill_status() == 0


def test_prefill_rejects_unsupported_widths(wm):
    """Prefill needs H, I and the shared width to be multiples of 256."""
    from winmoe_amd import synth
    cfg = _pf_cfg(E=8, K=2, H=384, I=256)
    sl = synth.build_layer(cfg, max_tokens=4)
    X = synth.make_hidden(cfg, tokens=4)
    with pytest.raises(wm.WinMoEError) as ei:
        sl.layer.prefill(X)
    assert ei.value.rc == wm._lib.WM_EINVAL


@pytest.mark.parametrize("types", [(Q4_K, Q5_K, Q6_K), (Q8_0, Q6_K, Q8_0)])
def test_prefill_rejects_unsupported_formats(wm, types):
    """Prefill refuses gate and up of different formats (WM_EINVAL, nothing
    launched); decode takes them."""
    from winmoe_amd import synth
    cfg = synth.LayerConfig("pf_fmt", E=8, K=2, H=512, I=256, types=types, tokens=1, x_dtype="bf16", seed=5)
    sl = synth.build_layer(cfg, max_tokens=4)
    X = synth.make_hidden(cfg, tokens=4)
    case(f"prefill refuses types={types}")
    with pytest.raises(wm.WinMoEError) as ei:
        sl.layer.prefill(X)
    assert ei.value.rc == wm._lib.WM_EINVAL
    assert np.isfinite(host(sl.layer.decode(X[0].float()))).all()


def test_prefill_rejects_two_pass_sizes(wm):
    """Both pass-size flags at once is an argument error."""
    from winmoe_amd import _lib, synth
    cfg = _pf_cfg(E=16, K=4, H=512, I=256, routing="zipf")
    sl = synth.build_layer(cfg, max_tokens=8)
    X = synth.make_hidden(cfg, tokens=8)
    ids = np.tile(np.arange(4, dtype=np.int32), (8, 1))
    w = np.full((8, 4), 0.25, np.float32)
    with pytest.raises(wm.WinMoEError) as ei:
        _prefill_flags(sl, X, ids, w, _lib.FLAG_PREFILL_PASS16 | _lib.FLAG_PREFILL_PASS32)
    assert ei.value.rc == _lib.WM_EINVAL


def test_prefill_forced_multi_pass_and_bad_ids(wm, orc):
    """Caller routing: one expert used by every token (three 32-pair passes),
    one invalid id (skipped, reported)."""
    from winmoe_amd import synth
    cfg = _pf_cfg(E=16, K=4, H=512, I=256, routing="zipf")
    T = 80
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg, tokens=T)
    rng = np.random.default_rng(5)
    ids = np.zeros((T, 4), np.int32)
    for t in range(T):
        ids[t, 1:] = rng.choice(np.arange(1, 16), 3, replace=False)
    ids[7, 2] = 99                                        # invalid
    w = rng.random((T, 4)).astype(np.float32)
    case(f"prefill forced T={T}")
    out = host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    for t in range(T):
        ok = (ids[t] >= 0) & (ids[t] < 16)
        _, _, ref = oracle_token(orc, sl, host(X[t].float()), ids=ids[t][ok], w=w[t][ok])
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    assert sl.layer.prefill_status() == 2                 # WM_STATUS_BAD_EXPERT_ID


def test_prefill_c5_full(wm, orc):
    """The 512-token, 512-expert, top-10 Q8_0 prefill with Zipf routing: a
    sample of tokens against the oracle, every token against the decode path
    with the same routing (a different route through the arithmetic)."""
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c5"]
    T = cfg.tokens
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg)
    ids, w = synth.forced_routes(cfg)
    case("prefill c5 full")
    out = host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    assert np.isfinite(out).all()
    case("prefill c5 full, passes of 16 and of 32 pairs")
    _check_pass_sizes(sl, X, ids, w, out)
    for t in (0, 1, 255, T - 1):
        case(f"prefill c5 oracle token={t}")
        _, _, ref = oracle_token(orc, sl, host(X[t].float()), ids=ids[t], w=w[t])
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    case("prefill c5 vs decode, all tokens")
    worst = 0.0
    for t in range(T):
        od = host(sl.layer.decode_forced(X[t].float(), dev(ids[t]), dev(w[t])))
        worst = max(worst, rel_l2(out[t], od))
    assert worst <= 1e-4, worst
    assert sl.layer.prefill_status() == 0


# K-quant experts in prefill: (gate = up, down) routed, shared or None, H.
# Routed and shared experts of different formats run as separate GEMM
# launches; H = 256 takes the two-block down items, 1024 the four-block ones;
# with passes of 16 pairs and H a multiple of 512, Q2_K .. Q4_K gate/up take
# stages of two super-blocks.
KQ_PREFILL = [
    ((Q4_K, Q6_K), (Q8_0, Q8_0), 1024),
    ((Q3_K, Q6_K), (Q4_K, Q8_0), 512),
    ((Q2_K, Q2_K), None, 1024),
    ((Q2_K, Q3_K), None, 256),
    ((Q5_K, Q5_K), (Q5_K, Q6_K), 1024),
    ((Q3_K, Q2_K), (Q4_K, Q4_K), 256),
    ((Q8_0, Q6_K), (Q2_K, Q8_0), 1024),
    ((Q4_K, Q4_K), (Q3_K, Q5_K), 256),
    ((Q6_K, Q4_K), None, 256),
    ((Q6_K, Q6_K), (Q8_0, Q6_K), 1024),
]


def _prefill_flags(sl, X, ids, w, flag):
    """The same forced prefill with `flag` added to the layer's flags (restored
    after)."""
    d = sl.layer.desc
    old = d.flags
    d.flags = old | flag
    try:
        return host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    finally:
        d.flags = old


def _check_pass_sizes(sl, X, ids, w, out):
    """Passes of 16 and of 32 pairs give `out` (the default choice's result)
    bit for bit."""
    from winmoe_amd import _lib
    for flag in (_lib.FLAG_PREFILL_PASS16, _lib.FLAG_PREFILL_PASS32):
        other = _prefill_flags(sl, X, ids, w, flag)
        assert np.array_equal(out.view(np.uint32), other.view(np.uint32)), flag


def _kq_routes(T, E, K, rng):
    """Every token uses expert 0 (passes of 32 + 32 + rest rows: both row
    tiles); the other slots are distinct random experts."""
    ids = np.zeros((T, K), np.int32)
    for t in range(T):
        ids[t, 1:] = rng.choice(np.arange(1, E), K - 1, replace=False)
    w = rng.random((T, K)).astype(np.float32)
    return ids, w


@pytest.mark.parametrize("gu,dn,sh,H", [(g, d, s, h) for (g, d), s, h in KQ_PREFILL],
                         ids=[f"{g}-{d}-{s}-h{h}" for (g, d), s, h in KQ_PREFILL])
def test_prefill_kquant_matches_oracle(wm, orc, gu, dn, sh, H):
    """Prefill with K-quant expert matrices (and a shared expert of another
    format) == the oracle token by token, with a 70-token batch whose
    expert 0 takes three passes (five in passes of 16 pairs: the same
    results bit for bit)."""
    from winmoe_amd import synth
    E, K, I, T = 24, 3, 512, 70
    cfg = synth.LayerConfig(f"pf_kq_{gu}_{dn}", E=E, K=K, H=H, I=I, types=(gu, gu, dn),
                            shared_types=(sh[0], sh[0], sh[1]) if sh else None, shared_inter=256 if sh else 0,
                            shared_gate_inp=sh is not None, tokens=1, routing="zipf", x_dtype="bf16", seed=13 + gu)
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg, tokens=T)
    ids, w = _kq_routes(T, E, K, np.random.default_rng(gu * 31 + dn))
    case(f"prefill kq gate/up={gu} down={dn} shared={sh} H={H} T={T}")
    out = host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    case(f"prefill kq gate/up={gu} down={dn} shared={sh} H={H} T={T}, passes of 16 and of 32 pairs")
    _check_pass_sizes(sl, X, ids, w, out)
    worst = 0.0
    for t in range(T):
        _, _, ref = oracle_token(orc, sl, host(X[t].float()), ids=ids[t], w=w[t])
        worst = max(worst, rel_l2(out[t], ref))
    print(f"worst rel-L2 vs oracle {worst:.3e}", flush=True)
    assert worst <= LAYER_TOL, worst
    assert sl.layer.prefill_status() == 0


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_prefill_kquant_full_layer(wm, orc, name):
    """A 512-token prefill through the full 512-expert layer of the Q4_K /
    Q6_K (shared Q8_0) and the Q2_K / Q3_K workloads with Zipf routing: a
    sample of tokens against the oracle, every token against the decode path
    with the same routing, and a second call bit-identical to the first, as
    is a call that takes the pairs in passes of 32 instead of 16."""
    import dataclasses
    from winmoe_amd import synth
    cfg = dataclasses.replace(synth.CONFIGS[name], tokens=512, routing="zipf", n_layers=1, x_dtype="bf16")
    T = cfg.tokens
    sl = synth.build_layer(cfg, max_tokens=T)
    X = synth.make_hidden(cfg)
    ids, w = synth.forced_routes(cfg)
    case(f"prefill {name} full")
    out = host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    again = host(sl.layer.prefill_forced(X, dev(ids), dev(w)))
    assert np.isfinite(out).all()
    assert np.array_equal(out.view(np.uint32), again.view(np.uint32))
    case(f"prefill {name} full, passes of 16 and of 32 pairs")
    _check_pass_sizes(sl, X, ids, w, out)
    for t in (0, 1, 255, T - 1):
        case(f"prefill {name} oracle token={t}")
        _, _, ref = oracle_token(orc, sl, host(X[t].float()), ids=ids[t], w=w[t])
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    case(f"prefill {name} vs decode, all tokens")
    worst = 0.0
    for t in range(T):
        od = host(sl.layer.decode_forced(X[t].float(), dev(ids[t]), dev(w[t])))
        worst = max(worst, rel_l2(out[t], od))
    print(f"worst rel-L2 vs decode {worst:.3e}", flush=True)
    assert worst <= 2e-4, worst
    assert sl.layer.prefill_status() == 0


# ------------------------------------------------------------------ GGUF boundary

@pytest.mark.parametrize("name", ["c1", "c3"])
def test_layer_from_gguf_matches_direct(wm, orc, tmp_path, name):
    """A layer written as a GGUF file (stacked [H, I, E] / [I, H, E] expert
    tensors, F32 router [H, E], shared expert) and mapped back with
    moe_layer_from_gguf decodes bit for bit like the same tensors handed over
    directly; the per-expert strides come from the tensor sizes."""
    from winmoe_amd import gguf, synth
    cfg = synth.CONFIGS[name]
    E = 24
    sl = synth.build_layer(cfg, E=E, max_tokens=4)
    H, I = cfg.H, cfg.I
    gt, ut, dt = cfg.types
    tensors = [("blk.3.ffn_gate_exps.weight", (H, I, E), gt, host(sl.gate).tobytes()),
               ("blk.3.ffn_up_exps.weight", (H, I, E), ut, host(sl.up).tobytes()),
               ("blk.3.ffn_down_exps.weight", (I, H, E), dt, host(sl.down).tobytes())]
    if sl.router is not None:
        tensors.append(("blk.3.ffn_gate_inp.weight", (H, E), 0, host(sl.router).tobytes()))
    if sl.shared is not None:
        sh = sl.shared
        Is = sh.inter
        tensors += [("blk.3.ffn_gate_shexp.weight", (H, Is), sh.types[0], host(sh.gate).tobytes()),
                    ("blk.3.ffn_up_shexp.weight", (H, Is), sh.types[1], host(sh.up).tobytes()),
                    ("blk.3.ffn_down_shexp.weight", (Is, H), sh.types[2], host(sh.down).tobytes())]
        if sh.gate_inp is not None:
            tensors.append(("blk.3.ffn_gate_inp_shexp.weight", (H,), 0, host(sh.gate_inp).tobytes()))
    p = str(tmp_path / "layer.gguf")
    gguf.write_gguf(p, {"general.architecture": "winmoe", "winmoe.expert_used_count": cfg.K}, tensors,
                    alignment=64)
    g = gguf.GGUFFile(p)
    L = gguf.moe_layer_from_gguf(g, 3, max_tokens=4)
    assert (L.H, L.I, L.E, L.K) == (H, I, E, cfg.K)
    X = synth.make_hidden(cfg, tokens=3)
    routes = synth.forced_routes(cfg, E=E, tokens=3) if cfg.routing != "router" else None
    for t in range(3):
        case(f"gguf {name} token={t}")
        if routes is None:
            a, b = host(L.decode(X[t])), host(sl.layer.decode(X[t]))
        else:
            ids, w = dev(routes[0][t]), dev(routes[1][t])
            a, b = host(L.decode_forced(X[t], ids, w)), host(sl.layer.decode_forced(X[t], ids, w))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
        if t == 0:
            # and against the oracle, on the bytes as read back from the file
            case(f"gguf {name} oracle token=0")
            xh = host(X[0])
            raw = {n[len("blk.3."):]: np.asarray(g.data(n)) for n, *_ in tensors}
            shared = None
            if sl.shared is not None:
                shared = (raw["ffn_gate_shexp.weight"], raw["ffn_up_shexp.weight"], raw["ffn_down_shexp.weight"])
            OL = orc.make_layer(H, I, E, cfg.K, cfg.types,
                                router=None if sl.router is None else
                                raw["ffn_gate_inp.weight"].view(np.float32).reshape(E, H),
                                gate=raw["ffn_gate_exps.weight"], up=raw["ffn_up_exps.weight"],
                                down=raw["ffn_down_exps.weight"], shared=shared,
                                sh_types=None if sl.shared is None else sl.shared.types,
                                sh_gate_inp=None if sl.shared is None or sl.shared.gate_inp is None else
                                raw["ffn_gate_inp_shexp.weight"].view(np.float32),
                                I_shared=0 if sl.shared is None else sl.shared.inter)
            fi = fw = None
            if routes is not None:
                fi, fw = routes[0][0], routes[1][0]
            oid, _, ref, _ = orc.moe_layer(OL, xh, fi, fw)
            if routes is None:
                assert host(L.trace()[0][0]).tolist() == oid.tolist()
            assert rel_l2(a, ref) <= LAYER_TOL, rel_l2(a, ref)
    assert L.status() == 0


@pytest.mark.parametrize("rtype", [1, Q8_0])
def test_gguf_router_f16_and_quantised(wm, orc, tmp_path, rtype):
    """A router stored as F16 or Q8_0 in the GGUF file is widened / dequantised
    exactly to fp32 at load; the layer then routes like the oracle on those
    fp32 weights."""
    import torch
    from winmoe_amd import gguf, synth
    cfg = synth.CONFIGS["c1"]
    E = 32
    sl = synth.build_layer(cfg, E=E, max_tokens=4)
    H, I = cfg.H, cfg.I
    W = host(sl.router)
    if rtype == 1:
        rbytes = W.astype(np.float16).tobytes()
        W32 = W.astype(np.float16).astype(np.float32)
    else:
        q = wm.quantize(sl.router.reshape(-1).contiguous(), Q8_0)
        rbytes = host(q).tobytes()
        W32 = orc.dequant(Q8_0, host(q)).reshape(E, H)
    gt, ut, dt = cfg.types
    tensors = [("blk.0.ffn_gate_exps.weight", (H, I, E), gt, host(sl.gate).tobytes()),
               ("blk.0.ffn_up_exps.weight", (H, I, E), ut, host(sl.up).tobytes()),
               ("blk.0.ffn_down_exps.weight", (I, H, E), dt, host(sl.down).tobytes()),
               ("blk.0.ffn_gate_inp.weight", (H, E), rtype, rbytes)]
    p = str(tmp_path / "router.gguf")
    gguf.write_gguf(p, {"general.architecture": "winmoe", "winmoe.expert_used_count": cfg.K}, tensors)
    L = gguf.moe_layer_from_gguf(gguf.GGUFFile(p), 0, max_tokens=4)
    assert np.array_equal(host(L.router).view(np.uint32), W32.view(np.uint32))
    X = synth.make_hidden(cfg, tokens=2)
    for t in range(2):
        case(f"gguf router type={rtype} token={t}")
        L.decode(X[t], step=t)
        oid, ow, _ = orc.router_topk(host(X[t]), W32, cfg.K)
        assert host(L.trace()[0][t]).tolist() == oid.tolist()
    del torch


# ------------------------------------------------------------------ RMSNorm in, residual out

@pytest.mark.parametrize("name,E,residual", [("c1", 64, True), ("c2", 40, True), ("c4", 24, True), ("c3", 24, True),
                                             ("c2", 512, True), ("c1", 1000, True), ("c2", 40, False)])
def test_fused_rmsnorm_and_residual(wm, orc, name, E, residual):
    """decode(h) with norm_w (and add_residual) == [h +] decode(rmsnorm(h)),
    the RMSNorm by the oracle (pinned to the reference's rmsnorm), bit for
    bit, with the same routing trace.  E=512 and E=1000 put two and four
    router rows on a workgroup of the persistent kernel (rows read the
    normalised x from LDS); c3 has a shared expert of another type (its x
    operand records are built separately).  The kernel adds the squares in
    its own order and falls back to the reference's index order when the two
    could round (float)(ss / H) differently, so the bar holds for every
    vector: the fifth token is one on a rounding boundary, where the two
    orders do disagree (rms_boundary_vector)."""
    import torch
    from winmoe_amd import synth
    from winmoe_amd.moe import MoELayer
    cfg = synth.CONFIGS[name]
    sl = synth.build_layer(cfg, E=E, max_tokens=8)
    c = sl.cfg
    g = torch.Generator(device="cuda").manual_seed(11)
    w = (1.0 + 0.1 * torch.randn(c.H, generator=g, device="cuda")).float()
    normed = MoELayer(c.H, c.I, E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types, shared=sl.shared, max_tokens=8,
                      norm_w=w, add_residual=residual)
    plain = synth.twin_layer(sl, multi_kernel=False)
    Hs = 3.0 * torch.randn(5, c.H, generator=g, device="cuda")
    Hs[4] = torch.from_numpy(rms_boundary_vector(c.H)).cuda()
    hb = host(Hs[4])
    fast, ref = rms_ss_kernel_order(hb), rms_ss_index_order(hb)
    assert np.float32(fast / c.H) != np.float32(ref / c.H)      # the orders disagree on token 4
    routes = synth.forced_routes(cfg, E=E, tokens=5) if cfg.routing != "router" else None
    for t in range(5):
        case(f"rmsnorm {name} E={E} token={t}")
        h = Hs[t].contiguous()
        hh = host(h)
        x = orc.rmsnorm(hh, host(w))
        if routes is None:
            a = host(normed.decode(h))
            b = host(plain.decode(dev(x)))
        else:
            ids, wt = dev(routes[0][t]), dev(routes[1][t])
            a = host(normed.decode_forced(h, ids, wt))
            b = host(plain.decode_forced(dev(x), ids, wt))
        want = hh + b if residual else b
        assert np.array_equal(a.view(np.uint32), want.view(np.uint32)), t
    ta, _ = normed.trace()
    tb, _ = plain.trace()
    assert np.array_equal(host(ta[:5]), host(tb[:5]))
    assert normed.status() == 0


def test_rmsnorm_rejected_off_the_persistent_path(wm):
    """The fused RMSNorm / residual belong to the persistent decode step: the
    per-phase and item-list paths and prefill refuse them (WM_EINVAL)."""
    import torch
    from winmoe_amd import _lib, synth
    from winmoe_amd.moe import MoELayer
    cfg = synth.CONFIGS["c1"]
    sl = synth.build_layer(cfg, max_tokens=4)
    c = sl.cfg
    w = torch.ones(c.H, device="cuda")
    for flags in (_lib.FLAG_MULTI_KERNEL, _lib.FLAG_ITEM_KERNEL):
        L = MoELayer(c.H, c.I, c.E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types, max_tokens=4, norm_w=w)
        L.desc.flags |= flags
        with pytest.raises(wm.WinMoEError) as ei:
            L.decode(torch.randn(c.H, device="cuda"))
        assert ei.value.rc == _lib.WM_EINVAL
    L = MoELayer(c.H, c.I, c.E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types, max_tokens=4, add_residual=True)
    with pytest.raises(wm.WinMoEError) as ei:
        L.decode(torch.randn(c.H, device="cuda"))
    assert ei.value.rc == _lib.WM_EINVAL
    with pytest.raises(wm.WinMoEError) as ei:
        L.prefill(torch.randn(4, c.H, device="cuda").to(torch.bfloat16))
    assert ei.value.rc == _lib.WM_EINVAL
