"""CPU checks of the f32-activation IQ3_S expert FFN (the reference's
fused_moe_iq3s, chimere-server/src/kernels/fused_moe.rs:101-311):

* the oracle's restatement in the library's fixed order (oracle/oracle.c,
  orc_fused_moe_iq3s) against an f64 evaluation built from the independent
  numpy IQ3_S decoder (tests/npref.py): dequantized weights times x in f64,
  silu, down projection, the weighted sum added to the prior output;
* a sign or scale mistake in the oracle's decode, a dropped expert, a
  swapped gate / up or a missing accumulate would each move the result far
  past the f32 rounding bound checked here;
* the C entry point's argument checks (no launch, no GPU needed)."""
import ctypes as C

import numpy as np
import pytest

import npref
import oracle as O
from chimere_amd import _lib


def silu64(g):
    return g / (1.0 + np.exp(-g))


def make(rng, H, F, E):
    q = lambda rows, cols: O.quantize(O.IQ3_S, (rng.standard_normal((E * rows, cols)) * 0.02).astype(np.float32))
    gate = q(F, H).reshape(E, -1)
    up = q(F, H).reshape(E, -1)
    down = q(H, F).reshape(E, -1)
    return gate, up, down


@pytest.mark.parametrize("H,F,E,K", [(256, 256, 3, 1), (1024, 256, 8, 5), (2048, 512, 12, 8)])
def test_oracle_against_f64(H, F, E, K):
    rng = np.random.default_rng(H + F + K)
    gate, up, down = make(rng, H, F, E)
    x = rng.standard_normal(H).astype(np.float32)
    ids = rng.permutation(E)[:K].astype(np.int32)
    wts = rng.uniform(0.05, 0.4, K).astype(np.float32)
    out0 = (rng.standard_normal(H) * 0.1).astype(np.float32)
    got = O.fused_moe_iq3s(x, gate, up, down, ids, wts, out0.copy(), H, F,
                           gate.shape[1], up.shape[1], down.shape[1])
    want = out0.astype(np.float64)
    for k, e in enumerate(ids):
        g = npref.dequant(21, gate[e], H) @ x.astype(np.float64)
        u = npref.dequant(21, up[e], H) @ x.astype(np.float64)
        h = silu64(g) * u
        want = want + float(wts[k]) * (npref.dequant(21, down[e], F) @ h)
    err = np.abs(got - want).max() / np.linalg.norm(want - out0)
    assert err < 2e-6, err
    # the f64 model tells a mistake apart: without the prior output, or with
    # one expert dropped, the result is off by far more than rounding
    assert np.abs(got - (want - out0)).max() / np.linalg.norm(want) > 1e-3
    if K > 1:
        part = out0.astype(np.float64)
        for k, e in enumerate(ids[:-1]):
            h = silu64(npref.dequant(21, gate[e], H) @ x) * (npref.dequant(21, up[e], H) @ x)
            part = part + float(wts[k]) * (npref.dequant(21, down[e], F) @ h)
        assert np.abs(got - part).max() / np.linalg.norm(want - out0) > 1e-3


def _err():
    L = _lib.lib()
    msg = L.chimere_hip_get_last_error_string().decode()
    return L.chimere_hip_get_last_error(), msg


def test_entry_point_validation():
    L = _lib.lib()
    assert L.chimere_fused_moe_iq3s_workspace_size(2048, 512, 8) == 8 * 512 * 4
    p = C.c_void_p(0x1000)
    ws = C.c_void_p(0x100000)
    good = dict(H=2048, F=512, bg=512 * 880, bu=512 * 880, bd=2048 * 220, K=8, wsb=1 << 20, ws=ws)

    def call(**kw):
        a = dict(good, **kw)
        L.chimere_fused_moe_iq3s(p, p, p, p, p, p, p, a["H"], a["F"], a["bg"], a["bu"], a["bd"], a["K"],
                                 a["ws"], a["wsb"], None)
        return _err()

    for bad in (dict(H=2000), dict(H=8192), dict(F=768), dict(F=0), dict(K=0), dict(K=17),
                dict(bg=100), dict(bd=2048 * 219), dict(bu=512 * 880 + 2)):
        assert call(**bad)[0] == 1, bad
    assert call(wsb=8 * 512 * 4 - 1)[0] == 3                 # workspace too small
    assert call(ws=C.c_void_p(0x100008))[0] == 3             # workspace not 16-byte aligned
    L.chimere_fused_moe_iq3s(None, p, p, p, p, p, p, 2048, 512, 512 * 880, 512 * 880, 2048 * 220, 8, ws,
                             1 << 20, None)
    code, msg = _err()
    assert code == 1 and "null" in msg
