"""Pins the CPU oracle: the reference's own known-answer tests, closed forms,
brute force on tiny inputs, and an independent numpy decode (tests/npref.py).
Runs on CPU only."""
import math
import os
import struct
import zlib

import numpy as np
import pytest

import oracle as O
import npref

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


# ------------------------------------------------------------------ IQ3_S grid

def test_iq3s_grid_golden():
    """Both copies of the 512-entry codebook equal the reference's table
    (gguf_loader.rs:941 == chimere_kernels.cu:66-131); crc32 of its
    little-endian bytes was taken from the reference text."""
    g_hip = npref.load_grid(os.path.join(ROOT, "chimere_amd", "csrc", "iq3s_grid.inc"))
    g_orc = npref.load_grid(os.path.join(ROOT, "oracle", "iq3s_grid.inc"))
    assert len(g_hip) == 512 and (g_hip == g_orc).all()
    assert zlib.crc32(g_hip.astype("<u4").tobytes()) == 0xF576E4F3
    b = g_hip.view(np.uint8)
    assert set(np.unique(b)) <= {1, 3, 5, 7, 9, 11, 13, 15}
    assert (np.diff(g_hip.astype(np.int64)) > 0).all()   # strictly increasing, no duplicates


# ------------------------------------------------------------------ f16 / exp

def test_f16_reference_kat():
    """ffi/src/lib.rs:851-866"""
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0x3800) == 0.5
    assert O.f16_to_f32(0xBC00) == -1.0
    assert O.f16_to_f32(0x0000) == 0.0
    assert math.copysign(1.0, O.f16_to_f32(0x8000)) == -1.0


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(v)) for v in h], np.float32)
    fin = np.isfinite(ref)
    assert (got[fin].view(np.uint32) == ref[fin].view(np.uint32)).all()
    assert np.isnan(got[np.isnan(ref)]).all()


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 17, 20000).astype(np.float32),
        # exact ties between two f16 values (RNE decides), subnormal range, overflow edge
        (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
        np.float32(2.0 ** -24) * np.arange(0, 64, 0.5, dtype=np.float32),
        np.array([65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8], np.float32)])
    got = np.array([O.f32_to_f16(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert (got == ref).all()


def test_exp_accuracy_and_exact_points():
    xs = np.linspace(-86, 88.7, 40001).astype(np.float32)
    got = np.array([O.exp(float(v)) for v in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 1.5e-7          # about one ulp
    assert O.exp(0.0) == 1.0
    assert O.exp(-87.0) == 0.0 and O.exp(-1000.0) == 0.0
    assert math.isinf(O.exp(89.0))
    # silu closed forms
    assert O.silu(0.0) == 0.0
    assert abs(O.silu(1.0) - 1.0 / (1.0 + math.exp(-1.0))) < 1e-7
    assert O.silu(-100.0) == 0.0 or abs(O.silu(-100.0)) < 1e-30


# ------------------------------------------------------------------ Q8_1

def _q8_1(x, npad=None):
    return O.quantize_q8_1(np.asarray(x, np.float32), npad or len(x))


def test_q8_1_ramp_kat():
    """lib.rs:966-1009 re-expressed for the 36-byte ggml layout: d = 32/127,
    q = round(x/d), s = sum x = 528."""
    x = np.arange(1, 33, dtype=np.float32)
    b = _q8_1(x)
    d, s, q = npref.q8_1_fields(b, 1)
    d32 = np.float32(32.0) / np.float32(127.0)
    assert d[0] == np.float32(d32).astype(np.float16).astype(np.float32)
    assert s[0] == 528.0
    assert (q[0] == np.round(x.astype(np.float64) / np.float64(d32)).astype(np.int64)).all()
    assert q[0, -1] == 127
    assert (np.abs(q[0] * d32 - x) < 0.3).all()


def test_q8_1_zeros_and_negatives():
    """lib.rs:1012-1044"""
    b = _q8_1(np.zeros(32, np.float32))
    assert (b == 0).all()
    b = _q8_1(-np.arange(1, 33, dtype=np.float32))
    d, s, q = npref.q8_1_fields(b, 1)
    assert d[0] > 0 and (q[0] <= 0).all() and s[0] <= 0


def test_q8_1_round_half_away_and_padding():
    # x/d lands exactly on .5 for these: amax = 127 -> d = 1
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:5] = [0.5, -0.5, 2.5, -2.5]
    d, s, q = npref.q8_1_fields(_q8_1(x), 1)
    assert d[0] == 1.0 and list(q[0, :5]) == [127, 1, -1, 3, -3]
    # ragged: 40 values padded to 64 -> second block holds 8 values then zeros
    y = np.arange(40, dtype=np.float32) - 20
    b = O.quantize_q8_1(y, 64)
    d, s, q = npref.q8_1_fields(b, 2)
    assert (q[1, 8:] == 0).all() and s[1] == np.float32(y[32:].sum())


def test_q8_1_sum_is_butterfly_order():
    """s = f16 of the sum in the 32-lane xor-butterfly order (masks 16..1,
    chimere_kernels.cu:1327-1333), not the sequential sum: pinned on an
    input where the two orders round differently."""
    rng = np.random.default_rng(7)
    for _ in range(2000):
        x = (rng.standard_normal(32) * np.float32(3.0) ** rng.integers(-8, 8, 32)).astype(np.float32)
        v = x.copy()
        for m in (16, 8, 4, 2, 1):
            v = (v + v[np.arange(32) ^ m]).astype(np.float32)
        seq = np.float32(0)
        for t in x:
            seq = np.float32(seq + t)
        s_bfly = np.float16(v[0])
        _, s, _ = npref.q8_1_fields(_q8_1(x), 1)
        assert s[0] == np.float32(s_bfly)
    # crafted: 2^25 at lane 0, -2^25 at lane 16, ones at lanes 1..15.  The
    # butterfly cancels the big pair first (s = 15); a sequential sum loses the
    # ones against 2^25 (s = 0).
    x = np.zeros(32, np.float32)
    x[0], x[16], x[1:16] = 2.0 ** 25, -(2.0 ** 25), 1.0
    _, s, _ = npref.q8_1_fields(_q8_1(x), 1)
    assert s[0] == 15.0


# ------------------------------------------------------------------ weight formats

def test_q8_0_known_block():
    """gguf_loader.rs:1765-1790 / lib.rs:868-887: d = 1.0, qs = 0..31."""
    blk = np.zeros(34, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:] = np.arange(32)
    assert (O.dequantize(O.Q8_0, blk, 32) == np.arange(32, dtype=np.float32)).all()


def test_q8_0_identity_gemv():
    """lib.rs:889-923: 32x32 with qs[row] = 1, d = 1, x = 1 -> y = 1, for the f64
    CPU path and for the Q8_1 path."""
    W = np.zeros((32, 34), np.uint8)
    W[:, 1] = 0x3C
    for r in range(32):
        W[r, 2 + r] = 1
    x = np.ones(32, np.float32)
    assert (O.gemv_q8_0_f64(W, x, 32, 32) == 1.0).all()
    y = O.gemv(O.Q8_0, W, O.quantize_q8_1(x, 32), 32, 32)
    # x=1 quantizes to q=127, d=f16(1/127): y = f16(1/127)*127
    assert np.allclose(y, np.float32(np.float16(1 / 127)) * 127, rtol=0, atol=0)


def test_q8_0_quantizer_roundtrip():
    """kv_q8_0.rs:49-89: amax element -> +-127, error <= d/2 per element."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    w = O.quantize(O.Q8_0, x)
    q, d = npref.levels(O.Q8_0, w, 256)
    amax = np.abs(x.reshape(64, 8, 32)).max(-1)
    assert (d == (amax / np.float32(127)).astype(np.float16).astype(np.float32)).all()
    assert (np.abs(q).reshape(64, 8, 32).max(-1) == 127).all()
    err = np.abs(npref.dequant(O.Q8_0, w, 256) - x)
    # half a step, plus the f16 rounding of d spread over |q| <= 127
    assert (err <= (np.repeat(d, 32, 1) * (0.5 + 127 * 2.0 ** -11) + 1e-6)).all()


def test_q4_0_layout_and_quantizer():
    """gguf_loader.rs:752-772: low nibble = element j, high = j+16, w = (n-8)d."""
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x3C]                         # d = 1
    blk[2:] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
    v = O.dequantize(O.Q4_0, blk, 32)
    assert (v[:16] == np.arange(16) - 8).all() and (v[16:] == 7 - np.arange(16)).all()
    rng = np.random.default_rng(4)
    x = rng.standard_normal((32, 512)).astype(np.float32)
    w = O.quantize(O.Q4_0, x)
    q, d = npref.levels(O.Q4_0, w, 512)
    xb = x.reshape(32, 16, 32)
    imax = np.abs(xb).argmax(-1)
    m = np.take_along_axis(xb, imax[..., None], -1)[..., 0]
    assert (d == (m / np.float32(-8)).astype(np.float16).astype(np.float32)).all()
    assert (np.take_along_axis(q.reshape(32, 16, 32), imax[..., None], -1) == -8).all()
    err = np.abs(npref.dequant(O.Q4_0, w, 512) - x)
    ad = np.abs(np.repeat(d, 32, 1)).astype(np.float64)
    # half a step (+ f16 rounding of d over |level| <= 8); values opposite to the
    # max element saturate at level 7, up to one full step away
    assert (err <= ad * (0.5 + 8 * 2.0 ** -11) + 0.5 * ad * (q == 7) + 1e-6).all()


def test_iq3s_decode_crafted_block():
    """gguf_loader.rs:1008-1142: index = qs | qh bit << 8, sign bit j of
    signs[4ib+l] negates element 8l+j, multiplier 1 + 2*nibble."""
    blk = np.zeros(110, np.uint8)
    blk[0:2] = [0x00, 0x3C]           # d = 1
    blk[74] = 0x81                    # sub-block 0, l=0: elements 0 and 7 negative
    blk[66] = 0x01                    # sub-block 0, l=0 first half: index 256
    blk[106] = 0x30                   # sub-block 1 multiplier 7
    blk[2 + 8 * 2 + 3] = 5            # sub-block 2, l=1, second half: index 5
    v = O.dequantize(O.IQ3_S, blk, 256)
    g256 = [(int(npref.GRID[256]) >> (8 * j)) & 255 for j in range(4)]
    g5 = [(int(npref.GRID[5]) >> (8 * j)) & 255 for j in range(4)]
    exp = np.ones(256)
    exp[0:4] = g256
    exp[0] = -exp[0]
    exp[7] = -1
    exp[32:64] = 7
    exp[64 + 12:64 + 16] = g5
    assert (v == exp).all()
    assert (v == npref.dequant(O.IQ3_S, blk, 256)[0]).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.IQ3_S])
def test_block_dots_match_numpy_decode(t):
    """Exact int32 block dots: C oracle == independent numpy decode."""
    rng = np.random.default_rng(t)
    ncols, nrows = 1024, 24
    W = rng.integers(0, 256, size=nrows * O.row_bytes(t, ncols), dtype=np.uint8)
    x = rng.standard_normal(ncols).astype(np.float32) * 3
    xq = O.quantize_q8_1(x)
    assert (O.block_dots(t, W, xq, ncols, nrows) == npref.block_dots(t, W, xq, ncols)).all()


def test_block_dots_synth251_fixture():
    """The reference's synthetic IQ3_S bytes (i % 251) and Q8_1 pattern
    (d = 0x1000, q = j % 5) from fused_gate_up.rs:386-412; block dots are
    checked against numpy and against the committed golden file."""
    ncols, nrows = 2048, 16
    W = (np.arange(nrows * ncols // 256 * 110) % 251).astype(np.uint8)
    xq = np.zeros(ncols // 32 * 36, np.uint8)
    for b in range(ncols // 32):
        xq[b * 36 + 1] = 0x10
        xq[b * 36 + 4:b * 36 + 36] = np.arange(32) % 5
    got = O.block_dots(O.IQ3_S, W, xq, ncols, nrows)
    assert (got == npref.block_dots(O.IQ3_S, W, xq, ncols)).all()
    gold = np.load(os.path.join(HERE, "golden", "iq3s_synth251_block_dots.npy"))
    assert (got == gold).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.IQ3_S])
def test_gemv_vs_f64_and_exact_invariants(t):
    rng = np.random.default_rng(10 + t)
    ncols, nrows = 2048, 64
    w = O.quantize(t, rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32))
    xq = O.quantize_q8_1(rng.standard_normal(ncols).astype(np.float32))
    y = O.gemv(t, w, xq, ncols, nrows)
    y64 = npref.gemv_f64(t, w, xq, ncols)
    assert np.linalg.norm(y - y64) / np.linalg.norm(y64) < 1e-6
    # brute force: dot of dequantized weights with dequantized activations
    dx, _, qx = npref.q8_1_fields(xq, ncols // 32)
    xd = (qx * dx[:, None].astype(np.float64)).reshape(-1)
    yb = npref.dequant(t, w, ncols) @ xd
    assert np.linalg.norm(y - yb) / np.linalg.norm(yb) < 1e-6
    # sign flip of the activations negates y exactly (sumi negates, fma is odd)
    xn = xq.copy().reshape(-1, 36)
    xn[:, 4:] = (-(xn[:, 4:].view(np.int8).astype(np.int16))).astype(np.int8).view(np.uint8)
    assert (O.gemv(t, w, xn.reshape(-1), ncols, nrows) == -y).all()
    # L=1 vs L=16 orders agree to rounding
    y1 = O.gemv(t, w, xq, ncols, nrows, L=1)
    assert np.linalg.norm(y - y1) / np.linalg.norm(y) < 1e-6
    # zero weight block contributes nothing: zero the whole matrix -> y = 0
    assert (O.gemv(t, np.zeros_like(w), xq, ncols, nrows) == 0).all()


def test_q4_0_all_eight_nibbles_zero():
    w = np.zeros((4, 18 * 4), np.uint8)
    w.reshape(4, 4, 18)[:, :, 0:2] = [0x00, 0x3C]
    w.reshape(4, 4, 18)[:, :, 2:] = 0x88
    xq = O.quantize_q8_1(np.linspace(-3, 3, 128).astype(np.float32))
    assert (O.block_dots(O.Q4_0, w, xq, 128, 4) == 0).all()


# ------------------------------------------------------------------ routing

def test_topk_reference_cases():
    """moe_forward.rs:322-403, fed as logits = log(p) (softmax(log p) = p)."""
    ids, w = O.topk_softmax(np.log(np.array([0.05, 0.60, 0.10, 0.25], np.float32)), 2)
    assert list(ids) == [1, 3]
    assert abs(w.sum() - 1) < 1e-6 and abs(w[0] / w[1] - 2.4) < 1e-4
    ids, w = O.topk_softmax(np.log(np.array([0.1, 0.8, 0.05, 0.05], np.float32)), 1)
    assert list(ids) == [1] and abs(w[0] - 1) < 1e-6
    ids, w = O.topk_softmax(np.zeros(4, np.float32), 2)          # all equal: lowest index first
    assert list(ids) == [0, 1] and np.allclose(w, 0.5, atol=1e-6)
    p = np.array([0.01, 0.50, 0.30, 0.07, 0.12], np.float32)
    for k in range(1, 6):
        ids, w = O.topk_softmax(np.log(p), k)
        assert abs(w.sum() - 1) < 1e-5
        assert list(ids) == list(np.argsort(-p, kind="stable")[:k])


def test_topk_random_against_sort():
    rng = np.random.default_rng(11)
    for _ in range(50):
        l = rng.standard_normal(256).astype(np.float32)
        ids, w = O.topk_softmax(l, 8)
        assert list(ids) == list(np.argsort(-l, kind="stable")[:8])
        p = np.exp(l.astype(np.float64) - l.max())
        ref = p[ids] / p[ids].sum()
        assert np.allclose(w, ref, rtol=2e-6, atol=0)


def test_router_order_and_accuracy():
    rng = np.random.default_rng(12)
    Wr = rng.normal(0, 0.02, (256, 2048)).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    l = O.router(Wr, x)
    ref = Wr.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(l - ref)) < 1e-5 * np.max(np.abs(ref)) + 1e-7
    # the order is the reference's: 256 strided fused-multiply-add lanes + halving tree
    acc = np.zeros(256, np.float64)
    a32 = np.zeros(256, np.float32)
    for j in range(2048):
        t = j & 255
        a32[t] = np.float32(np.float64(Wr[0, j]) * np.float64(x[j]) + np.float64(a32[t]))  # fma via f64 (exact product)
    v = a32.copy()
    for m in (128, 64, 32, 16, 8, 4, 2, 1):
        v[:m] = (v[:m] + v[m:2 * m]).astype(np.float32)
    assert np.float32(v[0]) == l[0]


# ------------------------------------------------------------------ MoE layer

def _moe_weights(rng, H, F, E, t):
    g = O.quantize(t, rng.normal(0, 0.02, (E * F, H)).astype(np.float32)).reshape(E, -1)
    u = O.quantize(t, rng.normal(0, 0.02, (E * F, H)).astype(np.float32)).reshape(E, -1)
    d = O.quantize(t, rng.normal(0, 0.02, (E * H, F)).astype(np.float32)).reshape(E, -1)
    return g, u, d


@pytest.mark.parametrize("t", [O.Q4_0, O.Q8_0, O.IQ3_S])
def test_moe_tiny_vs_dense_f64(t):
    """Brute force on a tiny layer (H=256, F=256, E=16, K=4): the quantized
    path tracks a float64 dense SwiGLU MoE on the dequantized weights."""
    rng = np.random.default_rng(20 + t)
    H, F, E, K = 256, 256, 16, 4
    Wr = rng.normal(0, 0.05, (E, H)).astype(np.float32)
    g, u, d = _moe_weights(rng, H, F, E, t)
    sh = tuple(a[0] for a in _moe_weights(rng, H, F, 1, t))
    gw = rng.normal(0, 0.05, H).astype(np.float32)
    x = rng.standard_normal((3, H)).astype(np.float32)
    out, ids, wts = O.moe(x, Wr, g, u, d, t, K, sh=sh, sh_type=t, sh_gate_w=gw)
    for m in range(3):
        lg = Wr.astype(np.float64) @ x[m]
        sel = np.argsort(-lg, kind="stable")[:K]
        assert list(ids[m]) == list(sel)
        p = np.exp(lg - lg.max())
        wr = p[sel] / p[sel].sum()
        assert np.allclose(wts[m], wr, rtol=1e-5)

        def ffn(G, U, D):
            gg = npref.dequant(t, G, H) @ x[m]
            uu = npref.dequant(t, U, H) @ x[m]
            hh = gg / (1 + np.exp(-gg)) * uu
            return npref.dequant(t, D, F) @ hh
        ref = sum(wr[k] * ffn(g[e], u[e], d[e]) for k, e in enumerate(sel))
        ref = ref + ffn(*sh) / (1 + np.exp(-(gw.astype(np.float64) @ x[m])))
        rel = np.linalg.norm(out[m] - ref) / np.linalg.norm(ref)
        assert rel < 0.03, rel   # activation (Q8_1) and weight quantization error


def test_moe_zero_input_and_extreme_k():
    """moe_forward.rs:405-460: zero input stays finite; k=1 and k=E work."""
    rng = np.random.default_rng(30)
    H, F, E = 256, 256, 8
    Wr = rng.normal(0, 0.05, (E, H)).astype(np.float32)
    g, u, d = _moe_weights(rng, H, F, E, O.Q4_0)
    out, ids, wts = O.moe(np.zeros((1, H), np.float32), Wr, g, u, d, O.Q4_0, 2)
    assert np.isfinite(out).all() and (out == 0).all() and list(ids[0]) == [0, 1]
    x = rng.standard_normal((1, H)).astype(np.float32)
    for k in (1, E):
        out, ids, wts = O.moe(x, Wr, g, u, d, O.Q4_0, k)
        assert np.isfinite(out).all() and abs(wts.sum() - 1) < 1e-5 and len(set(ids[0])) == k
