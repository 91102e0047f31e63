"""chimere_moe_ffn_decode_noalloc (static per-GPU scratch, no allocation)
against chimere_moe_ffn_decode (caller workspace) through the C ABI: equal
bits for outputs, routing indices and weights, on consecutive calls whose
second input is smaller (the scratch keeps the previous call's contents), and
a layer too large for the scratch is rejected before any launch."""
import numpy as np
import pytest
import torch

import oracle as O
from chimere_amd._lib import ChimereError
from test_gpu_moe import build, host, oracle_run

pytestmark = pytest.mark.gpu


def _both(layer, x):
    M, K = x.shape[0], layer.K
    res = []
    for fn in (layer.forward, layer.forward_noalloc):
        ids = torch.full((M, K), -1, dtype=torch.int32, device=x.device)
        wts = torch.zeros(M, K, device=x.device)
        out = torch.full_like(x, float("nan"))
        fn(x, out=out, ids=ids, wts=wts)
        res.append((host(out), host(ids), host(wts)))
    (ow, iw, ww), (on, in_, wn) = res
    assert (iw == in_).all() and (ww.view(np.uint32) == wn.view(np.uint32)).all()
    assert (ow.view(np.uint32) == on.view(np.uint32)).all()
    return on, in_, wn


@pytest.mark.parametrize("et,st,M0,M1", [
    (O.Q4_0, O.Q4_0, 8, 1),      # several-token launches, then the one-token kernels
    (O.IQ3_S, O.Q8_0, 4, 2),     # the IQ3_S model layer types
])
def test_noalloc_equals_workspace_entry(dev, et, st, M0, M1):
    print(f"noalloc et={et} st={st} M={M0} then {M1}", flush=True)
    layer = build(dev, 70 + et, et=et, st=st, gate_vec=True)
    g = torch.Generator(device=dev).manual_seed(71)
    x = torch.randn(M0, 2048, generator=g, device=dev)
    on, ig, wg = _both(layer, x)
    _both(layer, x[:M1].contiguous())      # second call, smaller input
    oo, io, _ = oracle_run(layer, x)       # and the first call's bits are the oracle's
    assert (ig == io).all() and (on.view(np.uint32) == oo.view(np.uint32)).all()


def test_noalloc_rejects_layer_beyond_scratch(dev):
    layer = build(dev, 72, H=4096, F=2048, E=16, K=8)
    x = torch.zeros(8, 4096, device=dev)
    with pytest.raises(ChimereError) as ei:
        layer.forward_noalloc(x)
    assert ei.value.code == 3
