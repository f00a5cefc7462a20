"""GPU tests of the boundary: the gpu_* shims' expert table (against the
semantics of gpu_offload.cu:582-673), the timeout path of the persistent
decode step, and decode steps issued on two streams at once.
"""
import numpy as np
import pytest

from golden.blocks import Q4_K, Q5_K, Q8_0
from helpers import rel_l2

pytestmark = pytest.mark.gpu

LAYER_TOL = 1e-3
MATVEC_TOL = 2e-4


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


def _expert_bytes(wm, seed, H, I, types):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [host(wm.quantize(torch.randn(r * c, generator=g, device="cuda") * 0.02, t))
            for t, r, c in ((types[0], I, H), (types[1], I, H), (types[2], H, I))]


def test_shim_expert_down(wm, orc):
    """gpu_expert_down: the down projection of a host activation vector with
    the slot's down matrix (gpu_offload.cu:700-712); -1 for an empty slot."""
    L = wm.load()
    H, I = 4096, 1024
    mats = _expert_bytes(wm, 3, H, I, (Q4_K, Q4_K, Q5_K))
    act = np.random.default_rng(4).standard_normal(I).astype(np.float32)
    case("gpu_expert_down")
    assert L.gpu_init() == 0
    slot = L.gpu_cache_expert(0, 7, mats[0].ctypes.data, mats[0].size, mats[1].ctypes.data, mats[1].size,
                              mats[2].ctypes.data, mats[2].size)
    assert slot >= 0
    y = np.zeros(H, np.float32)
    assert L.gpu_expert_down(slot, act.ctypes.data, I, y.ctypes.data, H) == 0
    assert rel_l2(y, orc.matvec(Q5_K, mats[2], act, H, I)) <= MATVEC_TOL
    assert L.gpu_expert_down(slot + 1, act.ctypes.data, I, y.ctypes.data, H) == -1
    L.gpu_shutdown()


def test_shim_limit_and_round_robin_eviction(wm, orc):
    """The expert table's contract: capacity 300 by default (MAX_GPU_EXPERTS),
    gpu_set_expert_limit clamps to at least 1, slots fill in order, the 301st
    insert recycles slot 0 and the next one slot 1 (round robin), a lowered
    limit leaves the cursor where it was (the next recycle takes it, then it
    wraps), a recycled expert is no longer found, ids past 80 layers x 1024 experts are refused,
    and a recycled slot computes with its new expert's bytes."""
    L = wm.load()
    H, I = 256, 256
    a = _expert_bytes(wm, 11, H, I, (Q8_0, Q8_0, Q8_0))
    b = _expert_bytes(wm, 12, H, I, (Q8_0, Q8_0, Q8_0))
    x = np.random.default_rng(5).standard_normal(H).astype(np.float32)

    def put(layer, eid, m):
        return L.gpu_cache_expert(layer, eid, m[0].ctypes.data, m[0].size, m[1].ctypes.data, m[1].size,
                                  m[2].ctypes.data, m[2].size)

    case("expert table: 302 inserts")
    assert L.gpu_init() == 0
    assert L.gpu_expert_cache_count() == 0
    slots = [put(e // 100, e % 100, a) for e in range(300)]
    assert slots == list(range(300))
    assert L.gpu_expert_cache_count() == 300
    assert L.gpu_find_cached_expert(0, 0) == 0 and L.gpu_find_cached_expert(2, 99) == 299
    assert put(5, 5, b) == 0                       # the 301st insert recycles slot 0
    assert L.gpu_find_cached_expert(0, 0) == -1 and L.gpu_find_cached_expert(5, 5) == 0
    assert put(5, 6, a) == 1                       # then slot 1
    assert L.gpu_find_cached_expert(0, 1) == -1 and L.gpu_expert_cache_count() == 300
    out = np.zeros(H, np.float32)
    assert L.gpu_expert_ffn_fused(0, x.ctypes.data, H, I, out.ctypes.data) == 0
    assert rel_l2(out, orc.expert_ffn(b[0], Q8_0, b[1], Q8_0, b[2], Q8_0, x, H, I)) <= LAYER_TOL
    assert put(80, 0, a) == -1 and put(0, 1024, a) == -1 and put(-1, 0, a) == -1
    # clamps to 1; the cursor is left where it was (slot 2, gpu_offload.cu:582-623),
    # so the next insert recycles slot 2, then the cursor wraps to 0 for good
    L.gpu_set_expert_limit(0)
    assert put(6, 1, a) == 2 and put(6, 2, a) == 0 and put(6, 3, a) == 0
    assert L.gpu_find_cached_expert(6, 1) == 2 and L.gpu_find_cached_expert(6, 2) == -1
    assert L.gpu_find_cached_expert(6, 3) == 0
    assert L.gpu_vram_used_mb() > 0
    L.gpu_shutdown()
    assert L.gpu_is_initialized() == 0 and L.gpu_find_cached_expert(6, 2) == -1


def test_spin_probe_reports_timeout_and_recovers(wm, orc):
    """WM_FLAG_SPIN_PROBE makes every wait of the persistent step on another
    workgroup give up at its first unsuccessful poll: the step ends with
    WM_STATUS_SPIN_TIMEOUT, MoELayer.check() raises, and after reset() the
    same layer decodes correctly again."""
    from winmoe_amd import _lib, synth
    cfg = synth.CONFIGS["c2"]
    sl = synth.build_layer(cfg, E=512, max_tokens=4)
    X = synth.make_hidden(cfg, tokens=2)
    case("spin probe")
    sl.layer.desc.flags |= _lib.FLAG_SPIN_PROBE
    sl.layer.decode(X[0])
    assert sl.layer.status() & _lib.STATUS_SPIN_TIMEOUT
    with pytest.raises(wm.WinMoEError):
        sl.layer.check()
    sl.layer.desc.flags &= ~_lib.FLAG_SPIN_PROBE
    sl.layer.reset()
    out = host(sl.layer.decode(X[1]))
    assert sl.layer.check() == 0
    ids, w = (host(a) for a in sl.layer.trace())
    xh = host(X[1])
    oid, ow, _ = orc.router_topk(xh, host(sl.router), cfg.K)
    assert ids[0].tolist() == oid.tolist()
    # the output against a twin layer that never saw the probe
    twin = synth.twin_layer(sl, multi_kernel=True)
    ref = host(twin.decode(X[1]))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_two_streams_interleaved(wm):
    """Two layers (own workspaces) decoding on two streams, their launches
    interleaved: the library orders the persistent launches, both stay
    correct (bit-identical to the same tokens run one stream at a time) and
    neither reports a timeout."""
    import torch
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c2"]
    a = synth.build_layer(cfg, E=512, max_tokens=8, layer_index=0)
    b = synth.build_layer(cfg, E=512, max_tokens=8, layer_index=1)
    X = synth.make_hidden(cfg, tokens=8)
    ref_a = [host(a.layer.decode(X[t])) for t in range(8)]
    ref_b = [host(b.layer.decode(X[t])) for t in range(8)]
    a.layer.reset()
    b.layer.reset()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    oa = torch.empty(8, cfg.H, device="cuda")
    ob = torch.empty(8, cfg.H, device="cuda")
    torch.cuda.synchronize()
    case("two streams")
    for t in range(8):
        a.layer.decode(X[t], out=oa[t], step=t, stream=sa)
        b.layer.decode(X[t], out=ob[t], step=t, stream=sb)
    torch.cuda.synchronize()
    assert a.layer.check() == 0 and b.layer.check() == 0
    for t in range(8):
        assert np.array_equal(host(oa[t]).view(np.uint32), ref_a[t].view(np.uint32)), t
        assert np.array_equal(host(ob[t]).view(np.uint32), ref_b[t].view(np.uint32)), t


def test_decode_graph_replay(wm):
    """Decode steps captured into a HIP graph (the benchmark times such
    replays): every replay, with eager work and host synchronisations between
    replays, gives the eager results bit for bit, with the same trace."""
    import torch
    from winmoe_amd import synth
    cfg = synth.CONFIGS["c2"]
    sl = synth.build_layer(cfg, E=512, max_tokens=8)
    X = synth.make_hidden(cfg, tokens=4)
    eager = [host(sl.layer.decode(X[t], step=t)) for t in range(4)]
    ids_e = host(sl.layer.trace()[0][:4])
    outs = torch.empty(4, cfg.H, device="cuda")
    g = torch.cuda.CUDAGraph()
    case("decode graph capture")
    with torch.cuda.graph(g):
        for t in range(4):
            sl.layer.decode(X[t], out=outs[t], step=t)
    for r in range(3):
        outs.fill_(float("nan"))
        sl.layer.trace(check=False)[0][:4].fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert sl.layer.check() == 0
        for t in range(4):
            assert np.array_equal(host(outs[t]).view(np.uint32), eager[t].view(np.uint32)), (r, t)
        assert np.array_equal(host(sl.layer.trace()[0][:4]), ids_e), r
        host(sl.layer.decode(X[0], step=5))          # eager work between replays
