"""CPU-side checks of the library boundary and host logic (no GPU compute)."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import header_functions

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "winmoe_hip.h")


@pytest.fixture(scope="module")
def lib():
    from winmoe_amd import _lib
    return _lib.load()


def test_library_exports_every_header_symbol(lib):
    from winmoe_amd import _lib
    names = header_functions(HEADER)
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_block_tables_match_oracle(lib, orc):
    for t in (8, 10, 11, 12, 13, 14):
        assert lib.wm_block_bytes(t) == orc.BLOCK_BYTES[t]
        assert lib.wm_block_elems(t) == orc.BLOCK_ELEMS[t]
    assert lib.wm_block_bytes(16) == 0 and lib.wm_block_bytes(7) == 0


def test_bad_arguments_rejected_without_gpu(lib):
    from winmoe_amd import _lib
    assert lib.wm_dequant(16, None, 1, None, None) == _lib.WM_EINVAL         # IQ2_XXS not on this path
    assert lib.wm_quantize(8, None, 33, None, None) == _lib.WM_EINVAL        # not whole blocks
    d = _lib.LayerDesc()
    assert lib.wm_workspace_size(C.byref(d), 16) == _lib.WM_EINVAL
    assert lib.wm_router_topk(None, None, 4096, 512, 17, None, None, None, 0, None) == _lib.WM_EINVAL  # K > 16


def _host_quantize(lib, t, x):
    from winmoe_amd import _lib
    n = x.size
    out = np.zeros(n // _lib.BLOCK_ELEMS[t] * _lib.BLOCK_BYTES[t], np.uint8)
    assert lib.wm_quantize_host(t, x.ctypes.data, n, out.ctypes.data) == 0
    return out


@pytest.mark.parametrize("t,tol", [(8, 0.51 / 127), (12, 0.6 / 15), (13, 0.6 / 31), (14, 0.6 / 31), (10, 0.7 / 3),
                                   (11, 0.6 / 4)])
def test_quantiser_round_trip(lib, orc, t, tol):
    """quantise -> oracle dequantise: per-block error bounded by about half a level."""
    rng = np.random.default_rng(t)
    x = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    blocks = _host_quantize(lib, t, x)
    y = orc.dequant(t, blocks)
    ne = orc.BLOCK_ELEMS[t]
    xb, yb = x.reshape(-1, ne), y.reshape(-1, ne)
    span = np.abs(xb).max(axis=1, keepdims=True) * (2.0 if t in (12, 13, 10) else 1.0)
    err = np.abs(yb - xb) / span
    assert err.max() < tol * 2.5, err.max()
    corr = np.corrcoef(x, y)[0, 1]
    assert corr > {8: 0.9999, 12: 0.99, 13: 0.997, 14: 0.998, 10: 0.88, 11: 0.93}[t], corr


def test_quantiser_q8_0_matches_ggml_convention(lib, orc):
    x = np.linspace(-1, 1, 32, dtype=np.float32) * 3.0
    b = _host_quantize(lib, 8, x)
    d = b[0:2].view(np.float16)[0]
    assert d == np.float16(np.float32(3.0) / np.float32(127.0))
    q = b[2:].view(np.int8)
    assert q[0] == -127 and q[-1] == 127


def test_zipf_generators():
    from winmoe_amd import synth
    rng = np.random.default_rng(0)
    ids = synth.zipf_routing(512, 512, 3, rng, overlap=synth.OVERLAP)
    st = synth.routing_stats(ids, 512)
    assert all(len(set(r)) == 3 for r in ids.tolist())
    assert 0.30 <= st["mean_overlap"] <= 0.45, st
    ids10 = synth.zipf_routing(512, 512, 10, np.random.default_rng(1))
    st10 = synth.routing_stats(ids10, 512)
    assert all(len(set(r)) == 10 for r in ids10.tolist())
    assert st10["max_count"] >= 40 and st10["experts_touched"] > 400, st10
    assert 0.2 < st10["zipf_slope_top30"] < 0.6, st10
    w = synth.softmax_weights(8, 10, rng)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


def test_config_byte_counts():
    from winmoe_amd import synth
    c2 = synth.CONFIGS["c2"]
    assert c2.expert_bytes() == 13_369_344 and c2.shared_bytes() == 13_369_344
    c3 = synth.CONFIGS["c3"]
    assert c3.expert_bytes() == 8_159_232
    c4 = synth.CONFIGS["c4"]
    assert c4.expert_bytes() == 4_554_752
    c1 = synth.CONFIGS["c1"]
    assert c1.expert_bytes() == 3_342_336


def test_pool_ids_checked_against_the_source(lib):
    """ExpertPool refuses ids outside the host source's experts before it
    calls the library (which refuses them too, WM_EINVAL); a pool that does
    not exist is refused without a GPU."""
    from winmoe_amd import _lib
    from winmoe_amd.moe import ExpertPool
    assert ExpertPool._ids(None, [0, 3, 511], 512).tolist() == [0, 3, 511]
    with pytest.raises(ValueError):
        ExpertPool._ids(None, [0, 512], 512)
    with pytest.raises(ValueError):
        ExpertPool._ids(None, [-1, 2], 512)
    ids = np.array([1, 2], np.int32)
    assert lib.wm_pool_acquire(None, 0, ids.ctypes.data_as(C.POINTER(C.c_int32)), 2, 4, None, None, None, 0, 0, 0,
                               None, None) == _lib.WM_EINVAL
    assert lib.wm_pool_acquire_packed(None, 0, ids.ctypes.data_as(C.POINTER(C.c_int32)), 2, 4, None, 0, None,
                                      None) == _lib.WM_EINVAL


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and says so,
    before touching a device."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_bench_names_the_prefill_kernels_the_library_picks():
    """The bench line's kernel names follow the library's pass-size rule (16
    pairs up to 10 per expert for Q8_0, 4 for K-quants) and its
    two-super-block stages for Q2_K .. Q4_K gate/up."""
    import importlib.util
    import sys
    from winmoe_amd import synth
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    sys.modules["bench_mod"] = bench
    spec.loader.exec_module(bench)
    assert bench.prefill_gateup_kernel(synth.CONFIGS["c5"]).startswith("k_pf_gemm<1,1,2,Q8_0,16,1>")
    c3p = bench.prefill_gateup_kernel(synth.CONFIGS["c3p"])
    assert c3p.startswith("k_pf_gemm<1,1,2,Q4_K,16,2> + k_pf_gemm<1,1,2,Q8_0,16,1>")
