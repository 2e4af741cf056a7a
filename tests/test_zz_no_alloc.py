"""The allocation-free decode entry point (frt_moe_layer_forward_noalloc) against the workspace one
(frt_moe_layer_forward) through the C ABI: identical ids, weights and outputs on two calls in a row,
the second with a smaller window, and its refusals."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests import helpers as H

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _run(w, x, resid, noalloc):
    T = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    rd = None if resid is None else torch.from_numpy(np.ascontiguousarray(resid)).cuda()
    out = torch.full((T, w.n), float("nan"), dtype=torch.float32, device="cuda")
    ids = torch.full((T, w.K), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros((T, w.K), dtype=torch.float32, device="cuda")
    if noalloc:
        w.layer_obj.forward_noalloc(xd, out, T=T, resid=rd, ids=ids, wts=wts)
    else:
        w.layer_obj.forward(xd, out, T=T, resid=rd, ids=ids, wts=wts)
    torch.cuda.synchronize()
    return out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()


@pytest.mark.parametrize("cfg", [0, 2])
def test_noalloc_matches_workspace_entry(cfg):
    import flashrt_amd as F
    F.lib()
    kw = {}
    if cfg == 2:
        kw = dict(layer=4, bias=O.gen_zipf_bias(2, 4, H.E, H.ZIPF_S_STACK), norm_input=True)
    w = H.World(cfg=cfg, **kw)
    rng = np.random.default_rng(40 + cfg)
    # a 3-token window, then a single token (smaller input; the persistent single-token path)
    for T in (3, 1):
        x = (rng.standard_normal((T, H.N)) * 2).astype(np.float32)
        resid = x if cfg == 2 else None
        got = _run(w, x, resid, noalloc=True)
        ref = _run(w, x, resid, noalloc=False)
        for a, b in zip(got, ref):
            assert np.array_equal(a, b), (cfg, T)
        assert np.isfinite(got[0]).all()
        assert not F.noalloc_sync_error()   # no allocation-free call ran out of time


def test_noalloc_largest_decode_workspace_fits():
    """Every decode window the entry point takes (E <= 1024, n <= 4096, ff <= 1024, T <= 4,
    T * K <= 63) has a layer workspace within the static array."""
    import ctypes as C
    import flashrt_amd as F
    from flashrt_amd._lib import FrtMoeLayer
    worst = 0
    for E in (512, 1024):
        for n in (1024, 2048, 4096):
            for ff in (512, 1024):
                for T in (1, 3, 4):
                    for K in (10, 21, 32):
                        if T * K > 63:
                            continue
                        d = FrtMoeLayer(1, 4096, E, 1, 1, 0, 1, n, ff, K, 0)
                        worst = max(worst, F.lib().frt_moe_layer_workspace_bytes(C.byref(d), T))
    assert 0 < worst <= F.noalloc_scratch_bytes(), worst


def test_noalloc_refuses_prefill_sizes():
    import flashrt_amd as F
    w = H.World(cfg=0)
    x = torch.zeros((8, H.N), dtype=torch.float32, device="cuda")
    out = torch.zeros_like(x)
    with pytest.raises(F.FrtError) as e:
        w.layer_obj.forward_noalloc(x, out, T=8)
    assert e.value.code == -1
    assert "decode windows only" in str(e.value)
    assert F.noalloc_scratch_bytes() == 4 << 20
