"""GPU parity at the benchmark workloads' full sizes (512 experts, hidden 4096,
intermediate 1024) against the CPU oracle on the same bytes.

Bars as in test_gpu_parity: router ids exact, routing weights within 1 ulp
(the device softmax rounds e^x from fp64; the oracle's expf is within ~0.5
ulp),
layer outputs rel-L2 <= 1e-3 against the oracle's fp32 dequant + fp64 maths,
dequantised blocks bit-exact.
"""
import os

import numpy as np
import pytest

from golden.blocks import Q2_K, Q3_K, Q4_K, Q5_K, Q8_0
from helpers import rel_l2, same_bits_nan, ulp_diff

pytestmark = pytest.mark.gpu

LAYER_TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


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


class HostExperts:
    """Host copies of a synthetic layer's expert slices, fetched once each, and
    the oracle's MoE block for one token over them."""

    def __init__(self, sl):
        from winmoe_amd.moe import matrix_bytes
        c = sl.cfg
        self.sl = sl
        gt, ut, dt = c.types
        self.sizes = (matrix_bytes(gt, c.I, c.H), matrix_bytes(ut, c.I, c.H), matrix_bytes(dt, c.H, c.I))
        self.cache = {}
        self.router = None if sl.router is None else host(sl.router)
        sh = sl.shared
        self.shared = None if sh is None else (host(sh.gate), host(sh.up), host(sh.down))
        self.gate_inp = None if (sh is None or sh.gate_inp is None) else host(sh.gate_inp).astype(np.float64)

    def expert(self, e):
        if e not in self.cache:
            pg, pu, pd = self.sizes
            s = self.sl
            self.cache[e] = (host(s.gate[e * pg:(e + 1) * pg]), host(s.up[e * pu:(e + 1) * pu]),
                             host(s.down[e * pd:(e + 1) * pd]))
        return self.cache[e]

    def token(self, orc, x, ids=None, w=None):
        c = self.sl.cfg
        H, I, K = c.H, c.I, c.K
        if ids is None:
            ids, w, _ = orc.router_topk(x, self.router, K)
        gt, ut, dt = c.types
        out = np.zeros(H)
        for k, e in enumerate(ids):
            g, u, d = self.expert(int(e))
            out += float(w[k]) * orc.expert_ffn(g, gt, u, ut, d, dt, x, H, I)
        if self.shared is not None:
            sh = self.sl.shared
            sg, su, sd = self.shared
            ys = orc.expert_ffn(sg, sh.types[0], su, sh.types[1], sd, sh.types[2], x, H, sh.inter or I)
            gate = 1.0
            if self.gate_inp is not None:
                gate = orc.lib().wmo_sigmoid(float(self.gate_inp @ x.astype(np.float64)))
            out += gate * ys
        return np.asarray(ids), np.asarray(w), out


def _decode_all(sl, X):
    """Every token of X through the layer's decode step (fused, persistent kernel)."""
    import torch
    outs = torch.empty_like(X)
    for t in range(X.shape[0]):
        sl.layer.decode(X[t], out=outs[t], step=t)
    return host(outs)


# ------------------------------------------------------------------ C2: 512 experts, top-10 + shared, Q8_0

@pytest.fixture(scope="module")
def c2(wm):
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c2"]
    sl = synth.build_layer(cfg, max_tokens=cfg.tokens)
    return sl, HostExperts(sl)


def test_c2_router_ids_every_token(wm, orc, c2):
    """All 256 decode tokens of the benchmark: ids exact and weights within 2
    ulp of the oracle router; 16 of them also against the oracle's output."""
    from winmoe_amd import synth
    sl, hx = c2
    cfg = sl.cfg
    X = synth.make_hidden(cfg)
    case("c2 full: 256 tokens")
    sl.layer.reset()
    out = _decode_all(sl, X)
    ids, w = (host(a) for a in sl.layer.trace())
    Xh = host(X)
    for t in range(cfg.tokens):
        oid, ow, _ = orc.router_topk(Xh[t], hx.router, cfg.K)
        assert ids[t].tolist() == oid.tolist(), t
        assert ulp_diff(w[t], ow).max() <= 1, t
    for t in range(0, cfg.tokens, cfg.tokens // 16):
        case(f"c2 full oracle output token={t}")
        _, _, ref = hx.token(orc, Xh[t], ids[t], w[t])
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    hits = host(sl.layer.hits())
    assert hits.sum() == cfg.tokens * cfg.K
    assert np.array_equal(hits, np.bincount(ids.reshape(-1), minlength=cfg.E))
    assert sl.layer.check() == 0


def test_c2_reference_layer0_input(wm, orc, c2):
    """The reference's own layer-0 MoE input (engine/runtime/moe_normed_L0.bin,
    winmoe_inference.c:1707; a real post-norm hidden state, rms 0.918) through
    the C2 layer."""
    sl, hx = c2
    x = np.fromfile(os.path.join(GOLDEN, "moe_normed_L0.bin"), dtype=np.float32)
    assert x.shape == (4096,)
    case("c2 reference L0 input")
    sl.layer.reset()
    out = host(sl.layer.decode(dev(x), step=0))
    ids, w = (host(a) for a in sl.layer.trace())
    oid, ow, ref = hx.token(orc, x)
    assert ids[0].tolist() == oid.tolist()
    assert ulp_diff(w[0], ow).max() <= 1
    assert rel_l2(out, ref) <= LAYER_TOL, rel_l2(out, ref)


def _seg_outlier_input(rng, H):
    x = rng.standard_normal(H).astype(np.float32)
    for s in range(H // 64):                       # one large value per 64-value segment
        x[64 * s + rng.integers(64)] = np.float32(rng.choice([-1, 1]) * 5.0e3)
    return x


@pytest.mark.parametrize("kind", ["outliers", "subnormals", "tiny_and_huge"])
def test_c2_activation_extremes(wm, orc, c2, kind):
    """Inputs the two-digit activation operand finds hardest: one outlier in
    every 64-value segment, subnormal entries mixed with normal ones, and
    segments of values ~1e-30 next to segments of values ~1e3."""
    sl, hx = c2
    rng = np.random.default_rng({"outliers": 1, "subnormals": 2, "tiny_and_huge": 3}[kind])
    H = sl.cfg.H
    if kind == "outliers":
        x = _seg_outlier_input(rng, H)
    elif kind == "subnormals":
        x = rng.standard_normal(H).astype(np.float32)
        idx = rng.choice(H, H // 8, replace=False)
        x[idx] = (rng.standard_normal(idx.size) * 1e-39).astype(np.float32)
        assert (np.abs(x[idx]) < np.finfo(np.float32).tiny).any()
    else:
        x = rng.standard_normal(H).astype(np.float32)
        x[:H // 2] *= np.float32(1e-30)
        x[H // 2:] *= np.float32(1e3)
    case(f"c2 activation extremes {kind}")
    sl.layer.reset()
    out = host(sl.layer.decode(dev(x), step=0))
    ids, w = (host(a) for a in sl.layer.trace())
    oid, ow, ref = hx.token(orc, x)
    assert ids[0].tolist() == oid.tolist()
    assert ulp_diff(w[0], ow).max() <= 1
    assert rel_l2(out, ref) <= LAYER_TOL, rel_l2(out, ref)


def test_c2_nonfinite_input_reports(wm, orc, c2):
    """A NaN in x makes every logit NaN: the reference's K-pass arg-max then
    picks expert 0 every time (nothing compares > -1e30) and its softmax is
    NaN (transformer.h:128-149).  The step reports degenerate routing and a
    non-finite weight, every output is NaN, and the next token is unaffected."""
    from winmoe_amd import _lib, synth
    sl, hx = c2
    x = host(synth.make_hidden(sl.cfg, tokens=2))
    bad = x[0].copy()
    bad[1234] = np.nan
    case("c2 NaN input")
    sl.layer.reset()
    out = host(sl.layer.decode(dev(bad), step=0))
    ids, w = (host(a) for a in sl.layer.trace())
    oid, ow, deg = orc.router_topk(bad, hx.router, sl.cfg.K)
    assert deg and ids[0].tolist() == oid.tolist() == [0] * sl.cfg.K
    assert np.isnan(w[0]).all() and np.isnan(out).all()
    st = sl.layer.check()
    assert st & _lib.STATUS_DEGENERATE_ROUTING and st & _lib.STATUS_NONFINITE_WEIGHT
    nxt = host(sl.layer.decode(dev(x[1]), step=1))
    _, _, ref = hx.token(orc, x[1])
    assert rel_l2(nxt, ref) <= LAYER_TOL


# ------------------------------------------------------------------ C3: top-3, Q4_K gate/up, Q6_K down, Q8_0 shared

def test_c3_full(wm, orc):
    """512 experts, top-3, Q4_K/Q6_K routed, Q8_0 shared expert with its gate:
    16 tokens (two router rows on each workgroup of the persistent kernel,
    the mixed-type x operand records)."""
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c3"]
    T = 16
    sl = synth.build_layer(cfg, max_tokens=T)
    hx = HostExperts(sl)
    X = synth.make_hidden(cfg, tokens=T)
    case("c3 full: 16 tokens")
    out = _decode_all(sl, X)
    ids, w = (host(a) for a in sl.layer.trace())
    Xh = host(X)
    for t in range(T):
        oid, ow, ref = hx.token(orc, Xh[t])
        assert ids[t].tolist() == oid.tolist(), t
        assert ulp_diff(w[t], ow).max() <= 1, t
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    assert sl.layer.check() == 0


# ------------------------------------------------------------------ C4: 8-layer Q2_K/Q3_K stack, forced Zipf routing

C4_TOKENS = 32


def _workers():
    """Host threads for the oracle (its C calls release the GIL)."""
    return max(1, min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def c4(wm):
    """The 8-layer, 512-expert, top-3 Q2_K/Q3_K stack, each layer with an
    RMSNorm and the residual add fused, and each layer's forced Zipf(0.456) /
    37.5 %-overlap routing for the benchmark's 512 tokens."""
    import torch
    from winmoe_amd import synth
    from winmoe_amd.moe import MoELayer
    cfg = synth.CONFIGS["c4"]
    g = torch.Generator(device="cuda").manual_seed(44)
    layers, hxs, routes, norms = [], [], [], []
    for li in range(cfg.n_layers):
        sl = synth.build_layer(cfg, layer_index=li, max_tokens=C4_TOKENS)
        c = sl.cfg
        nw = (1.0 + 0.1 * torch.randn(c.H, generator=g, device="cuda")).float()
        layers.append(MoELayer(c.H, c.I, c.E, c.K, None, sl.gate, sl.up, sl.down, c.types, max_tokens=C4_TOKENS,
                               norm_w=nw, add_residual=True))
        hxs.append(HostExperts(sl))
        routes.append(synth.forced_routes(cfg, layer_index=li))
        norms.append(host(nw))
    return cfg, layers, hxs, routes, norms


def test_c4_stack_full(wm, orc, c4):
    """32 tokens of the benchmark's trace through all 8 layers, chained as the
    reference chains its layers: h_{l+1} = h_l + moe_l(rmsnorm(h_l))
    (winmoe_inference.c:1659-1668, 2041), the RMSNorm and the residual add
    fused into each step.  Every (token, layer) is checked against the
    oracle's block on the GPU's own h_l, and the trace holds the forced ids
    and weights bit for bit."""
    import torch
    from concurrent.futures import ThreadPoolExecutor
    from winmoe_amd import synth
    cfg, layers, hxs, routes, norms = c4
    T, NL = C4_TOKENS, cfg.n_layers
    stats = synth.routing_stats(routes[0][0], cfg.E)
    assert 0.2 <= stats["mean_overlap"] <= 0.6, stats
    X = synth.make_hidden(cfg, tokens=T)
    hs = torch.empty(NL + 1, T, cfg.H, device="cuda")
    hs[0] = X
    case(f"c4 stack: {T} tokens x {NL} layers")
    for t in range(T):
        for li in range(NL):
            ids, w = routes[li]
            layers[li].decode_forced(hs[li, t], dev(ids[t]), dev(w[t]), out=hs[li + 1, t], step=t)
    H = host(hs)
    for li in range(NL):
        assert layers[li].check() == 0
        tid, tw = (host(a) for a in layers[li].trace())
        assert np.array_equal(tid[:T], routes[li][0][:T]) and np.array_equal(tw[:T].view(np.uint32),
                                                                               routes[li][1][:T].view(np.uint32))
        for e in set(routes[li][0][:T].reshape(-1).tolist()):
            hxs[li].expert(e)          # host copies fetched here, not in the workers

    def one(job):
        li, t = job
        x = orc.rmsnorm(H[li, t], norms[li])
        _, _, moe = hxs[li].token(orc, x, routes[li][0][t], routes[li][1][t])
        got = H[li + 1, t].astype(np.float64) - H[li, t].astype(np.float64)
        return li, t, rel_l2(got, moe)

    with ThreadPoolExecutor(max_workers=_workers()) as ex:
        errs = list(ex.map(one, [(li, t) for li in range(NL) for t in range(T)]))
    worst = max(errs, key=lambda r: r[2])
    assert worst[2] <= LAYER_TOL, worst
    for hx in hxs:
        hx.cache.clear()


def test_c4_dequant_every_touched_expert(wm, orc, c4):
    """Every block of the gate, up and down matrices of every expert that the
    benchmark's 512-token trace routes to, in each of the 8 layers (~400
    experts a layer), dequantises bit-exactly: per-block checksums of the fp32
    bit patterns (plain and position-weighted sums) from the device's
    wm_dequant against the oracle's, block by block."""
    import torch
    from winmoe_amd.moe import dequantize
    from winmoe_amd import _lib
    cfg, layers, hxs, routes, norms = c4
    gt, ut, dt = cfg.types
    nw = _workers()
    total = 0
    for li in range(cfg.n_layers):
        sl = hxs[li].sl
        pg, pu, pd = hxs[li].sizes
        touched = np.unique(routes[li][0].reshape(-1))
        assert touched.min() >= 0 and touched.max() < cfg.E
        case(f"c4 dequant: layer {li}, {touched.size} experts")
        idx = torch.from_numpy(touched.astype(np.int64)).cuda()
        for qt, src, per in ((gt, sl.gate, pg), (ut, sl.up, pu), (dt, sl.down, pd)):
            ne = _lib.BLOCK_ELEMS[qt]
            raw = src.view(cfg.E, per).index_select(0, idx).reshape(-1)
            pos = torch.arange(1, ne + 1, device="cuda", dtype=torch.int64)
            g1, g2 = [], []
            for c0 in range(0, touched.size, 64):
                part = raw[c0 * per:min(touched.size, c0 + 64) * per]
                u = dequantize(part, qt).view(torch.int32).to(torch.int64).bitwise_and_(0xFFFFFFFF).view(-1, ne)
                g1.append(u.sum(1))
                g2.append((u * pos).sum(1))
                del u
            g1 = host(torch.cat(g1))
            g2 = host(torch.cat(g2))
            s1, s2 = orc.dequant_block_sums(qt, host(raw), threads=nw)
            bad = np.flatnonzero((s1 != g1) | (s2 != g2))
            assert bad.size == 0, (li, qt, bad[:8], touched[bad[:8] // (per // orc.BLOCK_BYTES[qt])])
            total += s1.size
    print(f"[c4 dequant] {total} blocks checked", flush=True)


# ------------------------------------------------------------------ C5: batched prefill

@pytest.fixture(scope="module")
def c5(wm):
    import dataclasses
    from winmoe_amd import synth
    # the benchmark's layer plus a router (drawn after the experts, so the
    # expert bytes are the benchmark's)
    cfg = dataclasses.replace(synth.CONFIGS["c5"], routing="router")
    sl = synth.build_layer(cfg, max_tokens=cfg.tokens)
    return sl, HostExperts(sl)


def test_c5_router_every_token(wm, orc, c5):
    """512 bf16 tokens routed by the router: every token's ids exact and
    weights within 2 ulp of the oracle router, 16 outputs against the oracle."""
    from winmoe_amd import synth
    sl, hx = c5
    cfg = sl.cfg
    X = synth.make_hidden(cfg)
    case("c5 router prefill 512 tokens")
    out = host(sl.layer.prefill(X))
    ids, w = (host(a) for a in sl.layer.prefill_routing(cfg.tokens))
    Xf = host(X.float())
    for t in range(cfg.tokens):
        oid, ow, _ = orc.router_topk(Xf[t], hx.router, cfg.K)
        assert ids[t].tolist() == oid.tolist(), t
        assert ulp_diff(w[t], ow).max() <= 1, t
    for t in range(0, cfg.tokens, cfg.tokens // 16):
        case(f"c5 router prefill oracle token={t}")
        _, _, ref = hx.token(orc, Xf[t], ids[t], w[t])
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    assert sl.layer.prefill_status() == 0


def test_c5_zipf_oracle_and_twice(wm, orc, c5):
    """The benchmark's Zipf-routed batch: 16 tokens against the oracle, and a
    second run of the same batch bit-identical to the first (the grouping
    scatters pairs in atomic order; the per-expert order is then fixed)."""
    from winmoe_amd import synth
    sl, hx = c5
    cfg = sl.cfg
    X = synth.make_hidden(cfg)
    ids, w = synth.forced_routes(synth.CONFIGS["c5"])
    stats = synth.routing_stats(ids, cfg.E)
    assert stats["experts_touched"] == cfg.E and stats["max_count"] >= 50, stats
    case("c5 zipf prefill")
    di, dw = dev(ids), dev(w)
    a = host(sl.layer.prefill_forced(X, di, dw))
    b = host(sl.layer.prefill_forced(X, di, dw))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    Xf = host(X.float())
    for t in range(0, cfg.tokens, cfg.tokens // 16):
        _, _, ref = hx.token(orc, Xf[t], ids[t], w[t])
        assert rel_l2(a[t], ref) <= LAYER_TOL, (t, rel_l2(a[t], ref))
    assert sl.layer.prefill_status() == 0


# ------------------------------------------------------------------ the reference's own GPU type pair

def test_q4k_q5k_pair_through_the_layer(wm, orc):
    """Q4_K gate/up with Q5_K down -- the only types the reference's GPU path
    runs (gpu_offload.cu:730-744) -- through wm_moe_decode at 512 experts,
    with a Q4_K/Q5_K shared expert."""
    from winmoe_amd import synth
    cfg = synth.LayerConfig("e512_k8_h4096_i1024_q4k_q5k", E=512, K=8, H=4096, I=1024, types=(Q4_K, Q4_K, Q5_K),
                            shared_types=(Q4_K, Q4_K, Q5_K), shared_inter=1024, shared_gate_inp=True, tokens=6)
    sl = synth.build_layer(cfg, max_tokens=6)
    hx = HostExperts(sl)
    X = synth.make_hidden(cfg)
    case("q4k/q5k pair layer")
    out = _decode_all(sl, X)
    ids, w = (host(a) for a in sl.layer.trace())
    Xh = host(X)
    for t in range(cfg.tokens):
        oid, ow, ref = hx.token(orc, Xh[t])
        assert ids[t].tolist() == oid.tolist(), t
        assert rel_l2(out[t], ref) <= LAYER_TOL, (t, rel_l2(out[t], ref))
    assert sl.layer.check() == 0
