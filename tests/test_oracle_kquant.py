"""Pins the CPU oracle's ggml K-quant (Q4_K, Q5_K, Q6_K) and MXFP4 formats.

Checks, per type: crafted blocks built by an independent packer (ggml's
quantizer-side packing, tests/npref.py) dequantize to the closed form; the
oracle's dequant equals the numpy restatement of the reference's dequantizers
(gguf_loader.rs:839-917, 1165-1330); exact int32 block dots equal the numpy
ones; the GEMV in the (L=16, G=1) order is within 1e-6 of the order-free
float64 result and odd in x.  MXFP4 has no code in the reference tree: its
dequant is pinned against the OCP MX definition (E2M1 values times 2^(e-127)).
Runs on CPU only."""
import numpy as np
import pytest

import oracle as O
import npref

KQ = [O.Q4_K, O.Q5_K, O.Q6_K, O.MXFP4]


def _f32(x):
    return np.float32(x)


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K])
def test_k4_k5_crafted_blocks(t):
    """dequant(pack(fields)) == f32(d*sc) * q - f32(dmin*m), element by element."""
    rng = np.random.default_rng(t)
    for trial in range(4):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        if trial == 0:
            sc[:] = 63
            m[:] = 63                  # every high scale/min bit set
        qmax = 15 if t == O.Q4_K else 31
        q = rng.integers(0, qmax + 1, 256)
        d16 = np.float16(rng.uniform(1e-3, 2e-3)).view(np.uint16)
        dm16 = np.float16(rng.uniform(1e-4, 5e-4)).view(np.uint16)
        blk = (npref.pack_q4_k if t == O.Q4_K else npref.pack_q5_k)(d16, dm16, sc, m, q)
        d = np.uint16(d16).view(np.float16).astype(np.float32)
        dm = np.uint16(dm16).view(np.float16).astype(np.float32)
        want = np.array([_f32(d * _f32(sc[e // 32])) * _f32(q[e]) - _f32(dm * _f32(m[e // 32]))
                         for e in range(256)], np.float32)
        assert (O.dequantize(t, blk, 256) == want).all()
        assert np.allclose(npref.kq_dequant(t, blk, 256)[0], want, rtol=1e-6, atol=1e-9)


def test_q6_k_crafted_block():
    rng = np.random.default_rng(6)
    for trial in range(4):
        q = rng.integers(0, 64, 256)
        if trial == 0:
            q[:128] = 0
            q[128:] = 63               # extremes -32 and +31
        sc = rng.integers(-128, 128, 16)
        d16 = np.float16(rng.uniform(1e-4, 2e-4)).view(np.uint16)
        blk = npref.pack_q6_k(d16, sc, q)
        d = np.uint16(d16).view(np.float16).astype(np.float32)
        want = np.array([_f32(d * _f32(sc[e // 16])) * _f32(q[e] - 32) for e in range(256)], np.float32)
        assert (O.dequantize(O.Q6_K, blk, 256) == want).all()
        assert np.allclose(npref.kq_dequant(O.Q6_K, blk, 256)[0], want, rtol=1e-6, atol=1e-9)


def test_mxfp4_against_ocp_definition():
    """E2M1 code n: sign bit 3, magnitude {0, 0.5, 1, 1.5, 2, 3, 4, 6}[n & 7];
    E8M0 scale 2^(e-127); element j = low nibble of byte j, j+16 = high."""
    e2m1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    rng = np.random.default_rng(39)
    B = rng.integers(0, 256, (64, 17), dtype=np.uint8)
    B[:, 0] = rng.integers(100, 150, 64)
    B[0, 0], B[1, 0] = 1, 2            # low edge: half-scales 2^-127 (subnormal) and 2^-126
    got = O.dequantize(O.MXFP4, B.reshape(-1), 64 * 32).reshape(64, 32)
    for b in range(64):
        for j in range(32):
            nib = (B[b, 1 + j % 16] >> (4 * (j // 16))) & 15
            v = (-1.0 if nib & 8 else 1.0) * e2m1[nib & 7] * 2.0 ** (int(B[b, 0]) - 127)
            assert got[b, j] == np.float32(v), (b, j)
    assert (npref.kq_dequant(O.MXFP4, B.reshape(-1), 64 * 32).reshape(64, 32) == got).all()


@pytest.mark.parametrize("t", KQ)
def test_dequant_and_block_dots_match_numpy(t):
    rng = np.random.default_rng(100 + t)
    ncols, nrows = 1024, 12
    W = npref.rand_kq(t, nrows, ncols, rng)
    np.testing.assert_allclose(O.dequantize(t, W.reshape(-1), nrows * ncols).reshape(nrows, ncols),
                               npref.kq_dequant(t, W, ncols), rtol=1e-6, atol=1e-9)
    xq = O.quantize_q8_1(rng.standard_normal(ncols).astype(np.float32) * 2)
    assert (O.block_dots(t, W, xq, ncols, nrows) == npref.kq_block_dots(t, W, xq, ncols)).all()


@pytest.mark.parametrize("t", KQ)
def test_kq_gemv_vs_f64_and_odd(t):
    rng = np.random.default_rng(200 + t)
    ncols, nrows = 2048, 48
    W = npref.rand_kq(t, nrows, ncols, rng)
    xq = O.quantize_q8_1(rng.standard_normal(ncols).astype(np.float32))
    y = O.gemv(t, W, xq, ncols, nrows)
    y64 = npref.kq_gemv_f64(t, W, xq, ncols)
    assert np.linalg.norm(y - y64) / np.linalg.norm(y64) < 1e-6
    xn = xq.copy().reshape(-1, 36)
    xn[:, 4:] = (-(xn[:, 4:].view(np.int8).astype(np.int16))).astype(np.int8).view(np.uint8)
    assert (O.gemv(t, W, xn.reshape(-1), ncols, nrows) == -y).all()
    y1 = O.gemv(t, W, xq, ncols, nrows, L=1)
    assert np.linalg.norm(y - y1) / np.linalg.norm(y) < 1e-6


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K])
def test_k4_k5_min_term(t):
    """Quants all zero and scales zero: w = -dmin*m, so y = -sum_b dmin*m_b*dx_b*sum(q_x)."""
    rng = np.random.default_rng(300 + t)
    m = rng.integers(0, 64, 8)
    dm16 = np.float16(3e-4).view(np.uint16)
    blk = (npref.pack_q4_k if t == O.Q4_K else npref.pack_q5_k)(np.float16(1e-3).view(np.uint16), dm16,
                                                                 np.zeros(8, np.int64), m, np.zeros(256, np.int64))
    xq = O.quantize_q8_1(rng.standard_normal(256).astype(np.float32))
    assert (O.block_dots(t, blk, xq, 256, 1) == 0).all()
    dx, _, qx = npref.q8_1_fields(xq, 8)
    want = -sum(float(np.float16(3e-4)) * m[b] * float(dx[b]) * int(qx[b].sum()) for b in range(8))
    assert abs(float(O.gemv(t, blk, xq, 256, 1)[0]) - want) <= 1e-6 * max(1.0, abs(want))


def test_reference_all_001_input():
    """ggml_gpu.rs:1757-1903 feeds an all-0.01 input and accepts rel err < 0.02
    against a naive dequant kernel.  Here the bar is 1e-3 against the float64
    product of the dequantized weights with the UNquantized input: what is
    left is the Q8_1 rounding of the activation (d = 0.01/127 stored as f16,
    relative step 2^-11)."""
    rng = np.random.default_rng(7)
    ncols, nrows = 2048, 32
    x = np.full(ncols, 0.01, np.float32)
    xq = O.quantize_q8_1(x)
    for t in KQ:
        W = npref.rand_kq(t, nrows, ncols, rng)
        y = O.gemv(t, W, xq, ncols, nrows)
        yd = npref.kq_dequant(t, W, ncols) @ x.astype(np.float64)
        assert np.abs(y - yd).max() / np.abs(yd).max() < 1e-3, t
