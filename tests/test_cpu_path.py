"""The CPU baseline (oracle/cpu_path.c: the reference's CPU path structure
with AVX2 vec_dots, cs/ffi/ggml_iq3s_gemv.c:84-127) against the oracle: the
same int32 block dots, so GEMV rows agree to fp32 rounding (1e-5 of ||y||
for Q8_0 / Q4_0, 1e-4 for IQ3_S) and MoE layers route identically where the
top-k margin rule holds, with outputs within the same tolerances (the Q8_1
re-quantization of h turns an ulp-level gate/up difference into at most one
quantization step of one h value: 2e-3 of ||y||, as between the GPU's two fp32
orders)."""
import numpy as np
import pytest

import oracle as O
from routing_margin import topk_margin


def _w(t, rows, cols, rng):
    return O.quantize(t, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("t,tol", [(O.Q8_0, 1e-5), (O.Q4_0, 1e-5), (O.IQ3_S, 1e-4)])
@pytest.mark.parametrize("nthreads", [1, 4])
def test_cpu_gemv_vs_oracle(t, tol, nthreads):
    rng = np.random.default_rng(t)
    R, Cc = 300, 2048
    W = _w(t, R, Cc, rng)
    xq = O.quantize_q8_1(rng.standard_normal(Cc).astype(np.float32))
    y = O.cpu_gemv(t, W, xq, Cc, R, nthreads=nthreads)
    ref = np.ravel(O.gemv(t, W, xq, Cc, R))
    assert np.linalg.norm(y - ref) <= tol * np.linalg.norm(ref)
    # and the crafted extremes: all activations at -127 (the Q8_1 range: the
    # quantizer never emits -128) against weights with -128 bytes
    xq2 = xq.copy().reshape(-1, 36)
    xq2[:, 4:] = np.uint8(0x81)
    if t == O.Q8_0:
        W = W.copy().reshape(R, -1, 34)
        W[:, ::3, 2:10] = np.uint8(0x80)
        W = W.reshape(R, -1)
    y2 = O.cpu_gemv(t, W, xq2.reshape(-1), Cc, R, nthreads=nthreads)
    ref2 = np.ravel(O.gemv(t, W, xq2.reshape(-1), Cc, R))
    assert np.linalg.norm(y2 - ref2) <= tol * np.linalg.norm(ref2)


@pytest.mark.parametrize("et,st,tol", [(O.Q4_0, O.Q4_0, 2e-3), (O.IQ3_S, O.Q8_0, 2e-3)])
def test_cpu_moe_vs_oracle(et, st, tol):
    rng = np.random.default_rng(et + st)
    H, F, E, K, M = 1024, 256, 24, 8, 3
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    gate = np.stack([_w(et, F, H, rng).reshape(-1) for _ in range(E)])
    up = np.stack([_w(et, F, H, rng).reshape(-1) for _ in range(E)])
    down = np.stack([_w(et, H, F, rng).reshape(-1) for _ in range(E)])
    sh = tuple(_w(st, r, c, rng).reshape(-1) for r, c in ((F, H), (F, H), (H, F)))
    gw = (rng.standard_normal(H) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, H)).astype(np.float32)
    for m in range(M):
        assert topk_margin(O.router(router, x[m]), K) > 1e-4
    oo, io, wo = O.moe(x, router, gate, up, down, et, K, sh=sh, sh_type=st, sh_gate_w=gw)
    oc, ic, wc = O.cpu_moe(x, router, gate, up, down, et, K, sh=sh, sh_type=st, sh_gate_w=gw, nthreads=4)
    assert (io == ic).all()
    assert np.abs(wo - wc).max() <= 1e-5
    for m in range(M):
        assert np.linalg.norm(oc[m] - oo[m]) <= tol * np.linalg.norm(oo[m])
