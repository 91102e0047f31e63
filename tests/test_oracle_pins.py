"""Pins of the oracle functions that no reference test fixes directly:

* the IQ3_S encoder (orc_quantize_iq3_s): the reference tree holds no IQ3_S
  quantizer, only the layout and decode (cs/src/gguf_loader.rs:1008-1142).
  Its choices are checked against what the mathematics fixes: the super-block
  scale d = f16(amax / 465), the smallest odd multiplier 1 + 2s that covers
  the sub-block's largest magnitude, and, per group of 4, a brute-force
  search over all 512 codebook entries (the chosen entry has the smallest
  squared error in level space) with signs equal to the signs of x; an exact
  round trip of inputs built from codebook points.  The unpacking here uses
  the reference's shift form of the index (qh << (8 - 2l)) & 256, written
  apart from the oracle's and the numpy decoder's.
* the deterministic exponential: every float of [-87, 0] scanned, worst
  relative error and the size of its monotonicity steps.
* the top-k margin rule used by the GPU tests (tests/routing_margin.py)."""
import ctypes as C

import numpy as np
import pytest

import npref
import oracle as O
from routing_margin import EXP_ORDER_MARGIN, assert_topk_margin, topk_margin

GRID = npref.GRID
GLEV = np.stack([(GRID.astype(np.int64) >> (8 * j)) & 255 for j in range(4)], axis=1)   # [512, 4]


def unpack_iq3s(blk):
    """(d, mult[8], idx[8, 8], signs[8, 32]) of one 110-byte super-block."""
    d = np.float32(np.frombuffer(bytes(blk[0:2]), np.float16)[0])
    mult = np.array([1 + 2 * ((int(blk[106 + ib // 2]) >> (4 * (ib & 1))) & 15) for ib in range(8)])
    idx = np.zeros((8, 8), np.int64)
    neg = np.zeros((8, 32), bool)
    for ib in range(8):
        qh = int(blk[66 + ib])
        for l in range(4):
            idx[ib, 2 * l] = int(blk[2 + 8 * ib + 2 * l]) | ((qh << (8 - 2 * l)) & 256)
            idx[ib, 2 * l + 1] = int(blk[2 + 8 * ib + 2 * l + 1]) | ((qh << (7 - 2 * l)) & 256)
            sg = int(blk[74 + 4 * ib + l])
            for j in range(8):
                neg[ib, 8 * l + j] = (sg >> j) & 1 == 1
    return d, mult, idx, neg


def _inputs(seed):
    rng = np.random.default_rng(seed)
    x = [rng.normal(0, 0.02, 256 * 24).astype(np.float32),
         (rng.standard_t(2, 256 * 8) * 0.01).astype(np.float32)]        # heavy tails: outliers per sub-block
    z = rng.normal(0, 1, 256 * 4).astype(np.float32)
    z[256:512] *= 1e-3                                                 # tiny super-block (small f16 d)
    z[512 + 64:512 + 128] = 0.0                                        # all-zero sub-blocks
    z[768:1024:3] = 0.0
    x.append(z)
    return np.concatenate(x)


@pytest.mark.parametrize("seed", [1, 2])
def test_iq3s_encoder_bruteforce_optimal(seed):
    x = _inputs(seed)
    enc = O.quantize(O.IQ3_S, x)
    nsb = x.size // 256
    deq = npref.dequant(O.IQ3_S, enc, x.size)[0]
    worst_excess = 0.0
    for sb in range(nsb):
        v = x[sb * 256:(sb + 1) * 256].astype(np.float32)
        blk = enc[sb * 110:(sb + 1) * 110]
        amax = np.float32(np.abs(v).max())
        d_expect = np.float16(amax / np.float32(465.0))
        d, mult, idx, neg = unpack_iq3s(blk)
        if not float(d_expect) > 0:
            assert (blk == 0).all()
            continue
        assert np.float16(d) == d_expect, f"super-block {sb}: d"
        for ib in range(8):
            w = v[32 * ib:32 * ib + 32].astype(np.float64)
            sa = np.abs(w).max()
            m = int(mult[ib])
            # smallest odd multiplier whose top level 15 covers the largest magnitude
            cover = lambda mm: 15.0 * mm * float(d) >= sa * (1 - 1e-6)  # noqa: E731
            assert cover(m) or m == 31, f"{sb}/{ib}: multiplier {m} too small"
            assert m == 1 or not cover(m - 2) or abs(15.0 * (m - 2) * float(d) - sa) <= 1e-6 * sa, \
                f"{sb}/{ib}: multiplier {m} not the smallest"
            den = np.float64(np.float32(np.float32(d) * np.float32(m)))
            for l in range(4):
                for h in range(2):
                    e0 = 8 * l + 4 * h
                    target = np.abs(w[e0:e0 + 4]) / den
                    err = ((GLEV - target[None, :]) ** 2).sum(axis=1)
                    best = err.min()
                    got = err[idx[ib, 2 * l + h]]
                    worst_excess = max(worst_excess, got - best)
                    assert got <= best * (1 + 1e-5) + 1e-9, f"{sb}/{ib}/{l}/{h}: not the nearest codebook point"
            # signs are those of x (zero -> positive)
            assert (neg[ib] == (w < 0)).all(), f"{sb}/{ib}: signs"
            # the independent decoder sees the same values
            lev = np.array([GLEV[idx[ib, e // 4], e % 4] for e in range(32)]) * np.where(neg[ib], -1, 1)
            assert (deq[sb * 256 + 32 * ib:sb * 256 + 32 * ib + 32] == lev * m * np.float64(d)).all()
    assert worst_excess < 1e-3


def test_iq3s_encoder_exact_on_codebook_points():
    """Inputs built from codebook entries with a power-of-two d: the encoder
    must return exactly those entries, signs and multipliers."""
    rng = np.random.default_rng(5)
    has15 = np.nonzero((GLEV == 15).any(axis=1))[0]
    d = np.float32(2.0 ** -10)
    x = np.zeros(256 * 3, np.float32)
    want = []
    for sb in range(3):
        mults = rng.integers(0, 16, 8)
        mults[rng.integers(0, 8)] = 15           # amax = 15 * 31 * d: d = amax / 465 exactly
        for ib in range(8):
            gi = rng.integers(0, 512, 8)
            gi[rng.integers(0, 8)] = rng.choice(has15)   # the sub-block's largest level is 15
            sg = rng.integers(0, 2, 32).astype(bool)
            lev = np.array([GLEV[gi[e // 4], e % 4] for e in range(32)], np.float64)
            vals = np.where(sg, -lev, lev) * (1 + 2 * mults[ib]) * np.float64(d)
            x[sb * 256 + 32 * ib:sb * 256 + 32 * ib + 32] = vals.astype(np.float32)
            want.append((sb, ib, 1 + 2 * mults[ib], gi, sg))
    enc = O.quantize(O.IQ3_S, x)
    assert (npref.dequant(O.IQ3_S, enc, x.size)[0] == x.astype(np.float64)).all()
    for sb, ib, m, gi, sg in want:
        dd, mult, idx, neg = unpack_iq3s(enc[sb * 110:(sb + 1) * 110])
        assert dd == d and mult[ib] == m and (idx[ib] == gi).all() and (neg[ib] == sg).all()


def test_iq3s_encoder_zero_superblock():
    enc = O.quantize(O.IQ3_S, np.zeros(512, np.float32))
    assert (enc == 0).all()


def _exp_scan(lo, hi):
    L = O.lib()
    L.orc_exp_scan.restype = C.c_int64
    L.orc_exp_scan.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_int), C.POINTER(C.c_double)]
    step, rel = C.c_int(), C.c_double()
    bad = L.orc_exp_scan(lo, hi, C.byref(step), C.byref(rel))
    return bad, step.value, rel.value


def test_exp_every_float_in_softmax_range():
    """Every float in [-87, 0] (about 1.1e9 values; softmax arguments are
    l - max <= 0): relative error <= 1e-7 against the double exponential for
    x >= -86 (below that the result is flushed to 0), and the function never
    rises by more than one ulp from one float to the next -- it is monotone
    up to single-ulp rounding steps of the polynomial (2878 of them), which
    the top-k margin rule absorbs."""
    bad, step, rel = _exp_scan(-87.0, 0.0)
    assert rel < 1e-7
    assert step <= 1
    assert bad < 5000


def test_topk_margin_rule():
    lg = np.array([3.0, 1.0, 2.0, 0.0], np.float32)
    assert topk_margin(lg, 2) == pytest.approx(1.0)
    assert topk_margin(lg, 4) == np.inf
    tied = np.array([1.0, 1.0, 0.5], np.float32)
    assert topk_margin(tied, 1) == 0.0
    near = np.array([0.5, np.nextafter(np.float32(0.5), np.float32(0)), -1.0], np.float32)
    with pytest.raises(AssertionError):
        assert_topk_margin(near, 1)
    assert_topk_margin(lg, 3)
    # the rule is what keeps the oracle's selection equal to one made with the
    # exact exponential: sweep random rows that pass it
    rng = np.random.default_rng(0)
    for _ in range(200):
        row = rng.normal(0, 0.3, 256).astype(np.float32)
        if topk_margin(row, 8) <= EXP_ORDER_MARGIN:
            continue
        idx, _ = O.topk_softmax(row, 8)
        d = row.astype(np.float64) - row.max()
        assert (idx == np.argsort(-np.exp(d), kind="stable")[:8]).all()
