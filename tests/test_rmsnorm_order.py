"""The fused RMSNorm's sum of squares (CPU checks of the order rule).

The persistent decode step adds the squares in its own order (four fp64
chains per lane and an xor tree over the lanes) and the reference in index
order (attention.h:31-34).  The kernel takes its sum, forms q = ss / H and a
bound dq on the distance to the reference's quotient, and when q - dq and
q + dq round to different floats it adds the squares again in index order,
so its (float)(ss / H), and the scale, are the reference's.  These tests hold
the bound to what the arithmetic guarantees: on crafted vectors that sit on a
rounding boundary the two orders disagree and the rule falls back; over
random and near-boundary vectors every disagreement is caught by it, and it
falls back rarely."""
import numpy as np

from helpers import rms_boundary_vector, rms_scale, rms_ss_index_order, rms_ss_kernel_order


def falls_back(ss: float, H: int) -> bool:
    """The kernel's rule (wm_persist.hip, rmsnorm_lds)."""
    q = ss / H
    dq = q * ((2 * H + 8) * 2.0 ** -53) * 1.0625
    return np.float32(q - dq) != np.float32(q + dq)


def kernel_scale(h):
    H = len(h)
    ss = rms_ss_kernel_order(h)
    if falls_back(ss, H):
        ss = rms_ss_index_order(h)
    return rms_scale(ss, H)


def test_boundary_vector_needs_the_fallback(orc):
    for H in (2048, 4096):
        h = rms_boundary_vector(H)
        fast, ref = rms_ss_kernel_order(h), rms_ss_index_order(h)
        assert ref == 4097.0 ** 2                                   # every small square lost
        assert np.float32(fast / H) != np.float32(ref / H)           # the orders round differently
        assert falls_back(fast, H)
        w = np.ones(H, np.float32)
        want = orc.rmsnorm(h, w)                                     # the oracle (reference order)
        got = (h * kernel_scale(h)) * w
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_every_disagreement_falls_back():
    rng = np.random.default_rng(3)
    H = 1024
    disagree = caught = fallbacks = 0
    n = 400
    for i in range(n):
        kind = i % 4
        if kind == 0:
            h = rng.standard_normal(H).astype(np.float32)
        elif kind == 1:
            h = (rng.standard_t(2, H) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
        else:
            # near a boundary: one element at an odd 25-bit square root times
            # a power of two, the rest tiny with random sizes
            a = np.float32(rng.integers(2048, 2896) * 2 + 1) * np.float32(2.0 ** int(rng.integers(-8, 8)))
            tiny = np.float32(2.0 ** int(rng.integers(-20, -12)))
            h = (tiny * rng.uniform(0.5, 1.0, H)).astype(np.float32)
            h[int(rng.integers(0, H))] = a
        fast, ref = rms_ss_kernel_order(h), rms_ss_index_order(h)
        fb = falls_back(fast, H)
        fallbacks += fb
        if np.float32(fast / H) != np.float32(ref / H):
            disagree += 1
            caught += fb
        assert kernel_scale(h).view(np.uint32) == rms_scale(ref, H).view(np.uint32), i
    assert caught == disagree
    assert disagree > 0                    # the near-boundary family does reach the fallback
    # ordinary vectors almost never fall back
    plain = [rms_ss_kernel_order(rng.standard_normal(H).astype(np.float32)) for _ in range(200)]
    assert sum(falls_back(s, H) for s in plain) <= 2
