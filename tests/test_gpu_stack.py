"""Chained decode (wm_moe_decode_stack): several layers of one token in one
launch, layer l's input being layer l-1's output, against the same layers
entered one call each (wm_moe_decode / wm_moe_decode_forced), which the other
GPU tests hold to the oracle.  The bar is bit equality of every layer's
output, routing trace and status, over several tokens in a row (each launch
hands its outputs over in words tagged with that launch's epoch)."""
import dataclasses

import numpy as np
import pytest

from golden.blocks import Q4_K, Q5_K

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def wm():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import winmoe_amd
    winmoe_amd.load()
    return winmoe_amd


def host(t):
    return t.detach().cpu().numpy()


def case(msg):
    print(f"[case] {msg}", flush=True)


def _chain(cfg, NL, T, E, norm=True, forced=True, seed=7):
    """NL layers of cfg (E experts each), their RMSNorm weights, and per-layer
    forced routes for T tokens (or None: the layers' routers)."""
    import torch
    from winmoe_amd import synth
    from winmoe_amd.moe import MoELayer
    g = torch.Generator(device="cuda").manual_seed(seed)
    layers, routes = [], []
    for li in range(NL):
        sl = synth.build_layer(cfg, layer_index=li, max_tokens=T, E=E)
        c = sl.cfg
        nw = (1.0 + 0.1 * torch.randn(c.H, generator=g, device="cuda")).float() if norm else None
        layers.append(MoELayer(c.H, c.I, E, c.K, sl.router, sl.gate, sl.up, sl.down, c.types, shared=sl.shared,
                               max_tokens=T, norm_w=nw, add_residual=norm))
        if forced:
            ids, w = synth.forced_routes(cfg, layer_index=li, E=E, tokens=T)
            routes.append((torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()))
    return layers, (routes if forced else None)


def _twins(layers):
    """Second MoELayer objects over the same weights (their own workspaces)."""
    from winmoe_amd.moe import MoELayer
    out = []
    for m in layers:
        out.append(MoELayer(m.H, m.I, m.E, m.K, m.router, m.gate_exps, m.up_exps, m.down_exps, m.types,
                            shared=m.shared, max_tokens=m.max_tokens, norm_w=m.norm_w, norm_eps=m.desc.norm_eps,
                            add_residual=bool(m.desc.add_residual)))
    return out


def _compare(layers, routes, X, T):
    """Every token through the chain twice: layer by layer on one set of
    layer objects, chained in one call on their twins; outputs, traces and
    status equal bit for bit."""
    import torch
    from winmoe_amd.moe import decode_stack
    NL, H = len(layers), layers[0].H
    twins = _twins(layers)
    ref = torch.empty(T, NL, H, device="cuda")
    got = torch.empty(T, NL, H, device="cuda")
    for t in range(T):
        h = X[t]
        for li, m in enumerate(layers):
            r = routes[li] if routes else None
            if r is None:
                m.decode(h, out=ref[t, li], step=t)
            else:
                m.decode_forced(h, r[0][t], r[1][t], out=ref[t, li], step=t)
            h = ref[t, li]
        rr = [None if r is None else (r[0][t], r[1][t]) for r in routes] if routes else None
        decode_stack(twins, X[t], out=got[t], routes=rr, step=t)
    torch.cuda.synchronize()
    a, b = host(ref), host(got)
    bad = np.argwhere(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, ("first differing (token, layer, row)", bad[:4].tolist(),
                           "status", [tw.status() for tw in twins])
    for m, tw in zip(layers, twins):
        assert m.status() == 0 and tw.status() == 0, (m.status(), tw.status())
        ti, tw_ = (host(v) for v in m.trace())
        si, sw = (host(v) for v in tw.trace())
        assert np.array_equal(ti[:T], si[:T]) and np.array_equal(tw_[:T].view(np.uint32), sw[:T].view(np.uint32))
    return b


@pytest.mark.parametrize("NL", [1, 2, 8, 9, 11])
def test_stack_c4_layers_forced(wm, NL):
    """The C4 layer shape (Q2_K gate/up, Q3_K down, top-3, RMSNorm in,
    residual out, forced Zipf routes) at 64 experts: 1 layer (no chained
    launch), 2, 8 (one launch), 9 (a launch of 8, then the last layer on its
    own) and 11 (a launch of 8, then one of 3)."""
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c4"]
    T = 5
    case(f"stack c4 shape: {NL} layers x {T} tokens")
    layers, routes = _chain(cfg, NL, T, E=64)
    X = synth.make_hidden(cfg, tokens=T)
    _compare(layers, routes, X, T)


def test_stack_c4_full_experts(wm):
    """The benchmark's C4 stack: 8 layers of 512 experts, 6 tokens."""
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c4"]
    T = 6
    case("stack c4: 8 layers of 512 experts")
    layers, routes = _chain(cfg, 8, T, E=512)
    X = synth.make_hidden(cfg, tokens=T)
    _compare(layers, routes, X, T)


@pytest.mark.parametrize("norm", [True, False])
def test_stack_q8_router_layers(wm, norm):
    """Q8_0 layers routed by their own routers (the C1 shape, 64 experts),
    with and without RMSNorm / residual (without: each layer's output is its
    moe_out, the next layer's input), 3 layers x 4 tokens."""
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c1"]
    T = 4
    case(f"stack q8 router layers norm={norm}")
    layers, routes = _chain(cfg, 3, T, E=64, norm=norm, forced=False)
    X = synth.make_hidden(cfg, tokens=T)
    _compare(layers, routes, X, T)


def test_stack_mixed_routes_and_shared(wm):
    """The C3 layer shape (Q4_K/Q6_K experts, Q8_0 shared expert with its
    gate) at 64 experts: layer 0 routed by its router, layer 1 forced,
    layer 2 routed again."""
    import torch
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c3"]
    T = 4
    case("stack c3 shape, mixed routing")
    layers, _ = _chain(cfg, 3, T, E=64, forced=False)
    zr = dataclasses.replace(cfg, routing="zipf")
    ids, w = synth.forced_routes(zr, layer_index=1, E=64, tokens=T)
    routes = [None, (torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()), None]
    X = synth.make_hidden(cfg, tokens=T)
    _compare(layers, routes, X, T)


def test_stack_types_without_a_chained_instance(wm):
    """A format set with no chained instance (Q4_K/Q4_K/Q5_K) runs its
    layers one launch each inside the call, with the same results."""
    from winmoe_amd import synth
    cfg = dataclasses.replace(synth.CONFIGS["c4"], types=(Q4_K, Q4_K, Q5_K))
    T = 3
    case("stack fallback q4k/q5k")
    layers, routes = _chain(cfg, 3, T, E=64)
    X = synth.make_hidden(cfg, tokens=T)
    _compare(layers, routes, X, T)


def test_stack_layers_sharing_a_workspace(wm):
    """Two layers of a chain on one workspace (the layer tags and hand-off
    words live there) cannot share a launch: the call runs the chain one
    launch per layer instead, with the same outputs."""
    import torch
    from winmoe_amd import synth
    from winmoe_amd.moe import decode_stack
    cfg = synth.CONFIGS["c1"]
    T = 3
    case("stack with a shared workspace")
    layers, routes = _chain(cfg, 3, T, E=64)
    twins = _twins(layers)
    twins[1].ws = twins[0].ws
    X = synth.make_hidden(cfg, tokens=T)
    ref = torch.empty(T, 3, layers[0].H, device="cuda")
    got = torch.empty_like(ref)
    for t in range(T):
        h = X[t]
        for li, m in enumerate(layers):
            m.decode_forced(h, routes[li][0][t], routes[li][1][t], out=ref[t, li], step=t)
            h = ref[t, li]
        decode_stack(twins, X[t], out=got[t], routes=[(r[0][t], r[1][t]) for r in routes], step=t)
    torch.cuda.synchronize()
    a, b = host(ref), host(got)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert all(tw.status() == 0 for tw in twins)
