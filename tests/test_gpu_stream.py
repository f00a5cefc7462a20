"""GPU tests of host -> HBM expert streaming (wm_pool_*): experts held in
pinned host memory, made resident on demand in a pool of HBM slots
(the reference's miss path, winmoe_inference.c:1736-1789, and GPU cache
upload, gpu_offload.cu:590-659).  A step on the pool must agree with the
oracle run on the host bytes the pool copied from (layer tolerance), give the
same output, bit for bit, as the same step on the fully resident layer, and
the pool must replace slots as its contract says (free slots first, then the
least recently used one that no unreleased acquire holds)."""
import numpy as np
import pytest

from helpers import rel_l2

LAYER_TOL = 1e-3      # layer output rel-L2 vs the fp64 oracle

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


class LRUModel:
    """The pool's replacement rule restated: per acquire, the resident
    experts keep their slots and are held; a miss takes the lowest free slot,
    else the least recently used slot not held (since the last release, or
    by this call)."""

    def __init__(self, n):
        self.n, self.key, self.stamp, self.taken, self.clock = n, [None] * n, [0] * n, [False] * n, 0

    def acquire(self, layer, ids):
        keys = [(layer, int(e)) for e in ids]
        for k in keys:                      # the call's resident experts are held first
            if k in self.key:
                self.taken[self.key.index(k)] = True
        slots, misses = [], 0
        for k in keys:
            if k in self.key:
                s = self.key.index(k)
            else:
                free = [c for c in range(self.n) if self.key[c] is None and not self.taken[c]]
                if free:
                    s = free[0]
                else:
                    cand = [c for c in range(self.n) if not self.taken[c]]
                    s = min(cand, key=lambda c: self.stamp[c])
                self.key[s] = k
                misses += 1
            self.clock += 1
            self.stamp[s] = self.clock
            self.taken[s] = True
            slots.append(s)
        return slots, misses

    def release(self):
        self.taken = [False] * self.n


def _pool_setup(wm, name, E, n_slots):
    import torch
    from winmoe_amd import synth
    cfg = synth.CONFIGS[name]
    sl = synth.build_layer(cfg, E=E, max_tokens=64)
    c = sl.cfg
    gb, ub, db = (wm.matrix_bytes(t, r, k) for t, r, k in ((c.types[0], c.I, c.H), (c.types[1], c.I, c.H),
                                                             (c.types[2], c.H, c.I)))
    src = [t.view(E, -1).cpu().pin_memory() for t in (sl.gate, sl.up, sl.down)]
    assert [s.shape[1] for s in src] == [gb, ub, db]
    pool = wm.ExpertPool(n_slots, gb, ub, db)
    pl = pool.layer(c.H, c.I, c.K, c.types, shared=sl.shared, max_tokens=64)
    return cfg, sl, src, pool, pl


@pytest.mark.parametrize("name,E,n_slots", [("c3", 48, 8), ("c2", 40, 12)])
def test_pool_decode_matches_resident(wm, name, E, n_slots):
    """Tokens with Zipf routing through a pool smaller than the expert set
    (so slots are recycled under the steps): every output equals the
    resident layer's bit for bit, and hits / misses follow the replacement
    rule."""
    import torch
    from winmoe_amd import synth
    cfg, sl, src, pool, pl = _pool_setup(wm, name, E, n_slots)
    c = sl.cfg
    T = 32
    rng = np.random.default_rng(7)
    ids = synth.zipf_routing(T, E, c.K, rng, overlap=0.375)
    w = synth.softmax_weights(T, c.K, rng)
    X = synth.make_hidden(cfg, tokens=T)
    model = LRUModel(n_slots)
    outs = torch.empty(T, c.H, device="cuda")
    case(f"pool {name} E={E} slots={n_slots}: {T} tokens")
    want_slots = []
    for t in range(T):
        slots, misses = pool.acquire(0, ids[t], *src)
        ms, mm = model.acquire(0, ids[t])
        assert misses == mm, (t, misses, mm)
        want_slots.append(ms)
        pl.decode_forced(X[t], slots, torch.from_numpy(w[t]).cuda(), out=outs[t], step=t)
        pool.release()
        model.release()
        assert host(slots).tolist() == ms, t
    torch.cuda.synchronize()
    assert pl.check() == 0
    hits, misses, nbytes = pool.stats()
    assert hits + misses == T * c.K and misses > n_slots
    assert nbytes == misses * sum(s.shape[1] for s in src)
    for t in range(T):
        ref = host(sl.layer.decode_forced(X[t], torch.from_numpy(ids[t]).cuda(), torch.from_numpy(w[t]).cuda()))
        assert np.array_equal(host(outs[t]).view(np.uint32), ref.view(np.uint32)), t
    pool.close()


def test_pool_two_layers_and_limits(wm):
    """Two layers share one pool (their experts are distinct keys); more ids
    than slots, or acquires that together hold every slot without a
    release, are refused with WM_EINVAL and leave the pool usable."""
    import torch
    from winmoe_amd import synth
    cfg, sl, src, pool, pl = _pool_setup(wm, "c1", 16, 6)
    c = sl.cfg
    X = synth.make_hidden(cfg, tokens=4)
    w = torch.full((c.K,), 1.0 / c.K, device="cuda")
    case("pool: two layers, limits")
    a, m0 = pool.acquire(0, [1, 2, 3, 4], *src)
    pool.release()
    b, m1 = pool.acquire(1, [1, 2, 3, 4], *src)          # same ids, other layer: all misses
    pool.release()
    assert (m0, m1) == (4, 4)
    c_, m2 = pool.acquire(0, [1, 2, 3, 4], *src)         # slots of layer 0 partly recycled by layer 1
    assert m2 == 2
    with pytest.raises(wm.WinMoEError) as ei:
        pool.acquire(0, [5, 6, 7, 8, 9, 10, 11], *src)  # more ids than slots
    assert ei.value.rc == -2
    with pytest.raises(wm.WinMoEError) as ei:
        pool.acquire(0, [5, 6, 7], *src)                # 4 held + 3 new > 6 slots
    assert ei.value.rc == -2
    pool.release()
    s, _ = pool.acquire(0, [1, 2, 3, 4], *src)
    out = host(pl.decode_forced(X[0], s, w))
    pool.release()
    ref = host(sl.layer.decode_forced(X[0], torch.tensor([1, 2, 3, 4], dtype=torch.int32, device="cuda"), w))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    pool.close()


@pytest.mark.parametrize("name,n_slots,packed", [("c2", 24, False), ("c3", 12, True), ("c3", 12, False)])
def test_pool_vs_oracle_e512(wm, orc, name, n_slots, packed):
    """The C2 and C3 layers at E = 512 through a pool of a few slots (Zipf
    routing with overlap: slots are recycled under the steps), fed from
    pinned host tensors per part or from packed [gate | up | down] slot
    images (one copy per expert).  Tokens after several recycles are checked
    against the oracle run on those same host bytes with the same forced ids
    and weights; every token equals the resident layer bit for bit."""
    import torch
    from winmoe_amd import synth
    cfg, sl, src, pool, pl = _pool_setup(wm, name, 512, n_slots)
    c = sl.cfg
    T = 16
    rng = np.random.default_rng(11)
    ids = synth.zipf_routing(T, 512, c.K, rng, overlap=0.375)
    w = synth.softmax_weights(T, c.K, rng)
    X = synth.make_hidden(cfg, tokens=T)
    outs = torch.empty(T, c.H, device="cuda")
    image = pool.pack(*src) if packed else None
    case(f"pool {name} E=512 slots={n_slots} packed={packed}: {T} tokens")
    for t in range(T):
        if packed:
            slots, _ = pool.acquire_packed(0, ids[t], image)
        else:
            slots, _ = pool.acquire(0, ids[t], *src)
        pl.decode_forced(X[t], slots, torch.from_numpy(w[t]).cuda(), out=outs[t], step=t)
        pool.release()
    torch.cuda.synchronize()
    assert pl.check() == 0
    hits, misses, nbytes = pool.stats()
    assert misses > 2 * n_slots                     # slots were recycled
    assert nbytes == misses * sum(s_.shape[1] for s_ in src)
    # the oracle on the host bytes the pool read
    sh = sl.shared
    shared = None if sh is None else tuple(host(m) for m in (sh.gate, sh.up, sh.down))
    common = dict(shared=shared, sh_types=None if sh is None else sh.types,
                  sh_gate_inp=None if sh is None or sh.gate_inp is None else host(sh.gate_inp),
                  I_shared=0 if sh is None else sh.inter)
    if packed:
        flat = image.numpy().reshape(-1)
        sb = pool.slot_bytes
        OL = orc.make_layer(c.H, c.I, 512, c.K, c.types, gate=flat[pool.offsets[0]:], up=flat[pool.offsets[1]:],
                            down=flat[pool.offsets[2]:], strides=(sb, sb, sb), **common)
    else:
        OL = orc.make_layer(c.H, c.I, 512, c.K, c.types, gate=src[0].numpy(), up=src[1].numpy(),
                            down=src[2].numpy(), **common)
    for t in (3, 7, 11, 15):
        case(f"pool {name} oracle token={t}")
        _, _, ref, _ = orc.moe_layer(OL, host(X[t]), ids[t], w[t])
        got = host(outs[t])
        assert rel_l2(got, ref) <= LAYER_TOL, (t, rel_l2(got, ref))
    for t in range(T):
        res = host(sl.layer.decode_forced(X[t], torch.from_numpy(ids[t]).cuda(), torch.from_numpy(w[t]).cuda()))
        assert np.array_equal(host(outs[t]).view(np.uint32), res.view(np.uint32)), t
    pool.close()


def test_pool_refuses_ids_past_the_source(wm):
    """An id outside the host source's experts is refused with WM_EINVAL by
    the C-ABI (and with ValueError by ExpertPool) before any copy or state
    change; the pool stays usable."""
    import ctypes as C
    import torch
    from winmoe_amd import _lib
    cfg, sl, src, pool, pl = _pool_setup(wm, "c1", 16, 6)
    out = torch.empty(4, dtype=torch.int32, device="cuda")
    case("pool: id past the source")
    with pytest.raises(ValueError):
        pool.acquire(0, [1, 2, 16, 3], *src)
    bad = np.array([1, 2, 16, 3], np.int32)
    rc = _lib.load().wm_pool_acquire(pool._h, 0, bad.ctypes.data_as(C.POINTER(C.c_int32)), 4, 16,
                                     src[0].data_ptr(), src[1].data_ptr(), src[2].data_ptr(), src[0].stride(0),
                                     src[1].stride(0), src[2].stride(0), out.data_ptr(), None)
    assert rc == -2
    image = pool.pack(*src)
    rc = _lib.load().wm_pool_acquire_packed(pool._h, 0, bad.ctypes.data_as(C.POINTER(C.c_int32)), 4, 16,
                                            image.data_ptr(), image.stride(0), out.data_ptr(), None)
    assert rc == -2
    assert pool.stats() == (0, 0, 0)
    s, m = pool.acquire(0, [1, 2, 15, 3], *src)
    assert m == 4
    pool.release()
    pool.close()
