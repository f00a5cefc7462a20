"""wm_moe_decode_noalloc (workspace in the library's fixed device array)
against wm_moe_decode (caller workspace) through the C-ABI: the same kernels,
so the outputs and the routing agree bit for bit.  Two calls in a row, the
second on a smaller layer, so the array carries the first call's contents
into the second."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().cpu().numpy()


def _noalloc(L, layer, x):
    import torch
    out = torch.full((layer.H,), float("nan"), device="cuda")
    ids = torch.full((layer.K,), -1, dtype=torch.int32, device="cuda")
    w = torch.full((layer.K,), float("nan"), device="cuda")
    rc = L.wm_moe_decode_noalloc(C.byref(layer.desc), x.data_ptr(), out.data_ptr(), ids.data_ptr(), w.data_ptr(),
                                 C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, rc
    st = C.c_int32(-1)
    assert L.wm_noalloc_status(C.byref(st)) == 0
    return host(out), host(ids), host(w), st.value


def test_noalloc_matches_workspace_decode():
    import torch
    import winmoe_amd as wm
    from winmoe_amd import synth
    assert torch.cuda.is_available()
    L = wm.load()
    assert L.wm_noalloc_init() == 0
    assert L.wm_noalloc_scratch_bytes() == 3 * 1024 * 1024
    for name, E in (("c2", 512), ("c1", 64)):          # the second call is the smaller layer
        cfg = synth.CONFIGS[name]
        sl = synth.build_layer(cfg, E=E, max_tokens=4)
        x = synth.make_hidden(cfg, tokens=1)[0]
        print(f"[case] noalloc {name} E={E}", flush=True)
        out, ids, w, st = _noalloc(L, sl.layer, x)
        ref = host(sl.layer.decode(x, step=0))
        rid, rw = (host(a[0]) for a in sl.layer.trace())
        assert st == 0 and sl.layer.check() == 0
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), name
        assert ids.tolist() == rid.tolist() and np.array_equal(w.view(np.uint32), rw.view(np.uint32))


def test_noalloc_rejects_oversized_layer():
    """A layer whose decode workspace is past the array is refused (WM_EINVAL)
    before anything runs."""
    import winmoe_amd as wm
    from winmoe_amd import _lib
    L = wm.load()
    d = _lib.LayerDesc()
    d.hidden, d.inter, d.n_experts, d.top_k = 4096, 4096, 1024, 16
    d.gate_type = d.up_type = d.down_type = _lib.Q8_0
    d.flags = _lib.FLAG_TIMELINE                        # the timeline makes the workspace larger than the array
    assert L.wm_workspace_size(C.byref(d), 1) > L.wm_noalloc_scratch_bytes()
    rc = L.wm_moe_decode_noalloc(C.byref(d), C.c_void_p(16), C.c_void_p(16), None, None, None)
    assert rc == _lib.WM_EINVAL
