"""Pins of the oracle's Q4_0 s-form GEMV (ggml's block term
d_w * (sum(nib * q_x) * d_x - 8 * s_x), mul_mat_vec_q4_0_q8_1 reached in the
reference only through libllama, out of tree).

* an independent float64 evaluation of the same expression from the raw
  bytes (numpy unpacking of the Q4_0 and Q8_1 blocks, written apart from the
  oracle) agrees within fp32 rounding;
* against the exact integer form the difference is bounded by what the
  mathematics fixes: sum over blocks of 8 |d_w| |s_x - d_x * sum(q_x)| plus
  fp32 rounding;
* a hand-computed single-block case."""
import numpy as np
import pytest

import oracle as O


def f16(b):
    return np.frombuffer(np.asarray(b, np.uint8).tobytes(), np.float16).astype(np.float64)


def unpack_q4_0(row, nb):
    blk = row.reshape(nb, 18)
    d = f16(blk[:, :2].copy())
    lo, hi = blk[:, 2:] & 0xF, blk[:, 2:] >> 4
    nib = np.concatenate([lo, hi], axis=1).astype(np.int64)   # element j < 16: lo, j >= 16: hi
    return d, nib


def unpack_q8_1(xq, nb):
    blk = xq[:nb * 36].reshape(nb, 36)
    d = f16(blk[:, 0:2].copy())
    s = f16(blk[:, 2:4].copy())
    q = blk[:, 4:].view(np.int8).astype(np.int64)
    return d, s, q


@pytest.mark.parametrize("nrows,ncols,seed", [(64, 2048, 1), (33, 512, 2), (7, 4096, 3)])
def test_sform_f64_and_bound(nrows, ncols, seed):
    rng = np.random.default_rng(seed)
    W = O.quantize(O.Q4_0, rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32))
    x = (rng.standard_normal(ncols) * 1.7).astype(np.float32)
    xq = O.quantize_q8_1(x)
    nb = ncols // 32
    ys = O.gemv(O.Q4_0_SFORM, W, xq, ncols, nrows)
    ye = O.gemv(O.Q4_0, W, xq, ncols, nrows)
    dx, sx, qx = unpack_q8_1(xq, nb)
    ref = np.zeros(nrows)
    bound = np.zeros(nrows)
    for r in range(nrows):
        dw, nib = unpack_q4_0(W[r], nb)
        sumi = (nib * qx).sum(axis=1)
        ref[r] = (dw * (sumi * dx - 8 * sx)).sum()
        bound[r] = (8 * np.abs(dw) * np.abs(sx - dx * qx.sum(axis=1))).sum()
    n = np.linalg.norm(ref)
    assert np.linalg.norm(ys - ref) <= 2e-6 * n
    # the two forms differ by the s_x term's rounding, nothing else
    slack = 1e-5 * np.abs(ref).max()
    assert (np.abs(ys.astype(np.float64) - ye) <= bound + slack).all()
    assert (bound > 0).any()   # the forms do differ on these inputs


def test_sform_one_block_by_hand():
    # weight block: d = 0.5, every nibble 9; activation block from x (all of
    # its 32 quants known), so sum(nib * q) = 9 * sum(q)
    w = np.zeros(18, np.uint8)
    w[:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    w[2:] = 0x99
    x = np.linspace(-1.0, 1.0, 32).astype(np.float32)
    xq = O.quantize_q8_1(x)
    dx, sx, qx = unpack_q8_1(xq, 1)
    sumi = 9 * int(qx.sum())
    y = O.gemv(O.Q4_0_SFORM, w.reshape(1, 18), xq, 32, 1)[0]
    # fmaf(sumi, d_x, -8 s_x): the float64 value is exact here (a 16-bit
    # integer times an f16, plus an f16), so one rounding to float32 is fmaf;
    # the final fmaf(0.5, inner, 0) is exact
    inner = np.float32(float(sumi) * float(dx[0]) - 8.0 * float(sx[0]))
    assert y == np.float32(0.5 * float(inner)), (y, inner)
