"""The host-side expert path ("ncmoe"): chimere-server/src/qwen35_model/moe_ffn.rs:1507-1591
over its ggml wrapper chimere-server/ffi/ggml_iq3s_gemv.c:33-127.

ggml (ik_llama.cpp) is not in the reference tree and the reference holds no
test vectors for this path, so the oracle's restatement is pinned here by
what the mathematics fixes:

* Q8_K quantization: hand-computed blocks (which element sets the scale,
  round-half-even on exact ties, the zero block), and for random data the
  invariants |x - d q| <= |d| / 2, q = -127 at the scale-setting element,
  bsums = sums of 16 quants;
* the IQ3_S x Q8_K dot: a single super-block equals
  f32(f32(d_w d_y) * isum) exactly, with isum from the numpy decoder
  (tests/npref.py) and the quants read back from the bytes; several
  super-blocks stay within the sequential-rounding bound of the float64 sum;
* the GEMV tracks the float product W x within the quantization bound;
* the expert loop: K = 1 composes GEMV -> SwiGLU -> GEMV exactly as the Rust
  code; power-of-two weights make the weighted sum exact, so its order is
  checked bit for bit; a float64 evaluation bounds the whole token.

The product library (libchimere_cpu.so) is then held bit-exact to the oracle:
integer super-block sums are exact in both, and the float steps are the same
sequence, so no tolerance is needed.  The exported names are those of
include/chimere_cpu.h."""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import npref
import oracle as O
from chimere_amd import cpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EPS = np.finfo(np.float32).eps


def q8k_fields(y, nb):
    B = np.asarray(y, np.uint8).reshape(nb, 296)
    d = B[:, 0:4].copy().view(np.float32).ravel()
    s = B[:, 4:8].copy().view(np.float32).ravel()
    q = B[:, 8:264].view(np.int8).astype(np.int64)
    bs = B[:, 264:296].copy().view(np.int16).astype(np.int64)
    return d, s, q, bs


def iq3s_bank(rng, E, rows, cols, scale=0.02):
    return np.stack([O.quantize(O.IQ3_S, rng.normal(0, scale, rows * cols).astype(np.float32)) for _ in range(E)])


# ---------------------------------------------------------------- Q8_K pins

def test_q8K_hand_block_ties_and_scale_element():
    m = np.float32(-127.0 / 64.0)                      # iscale = -127 / m = 64 exactly
    x = np.zeros(256, np.float32)
    x[0] = m
    x[1] = -m                                          # same magnitude later: does not set the scale
    x[2], x[3], x[4], x[5] = 5 / 128, 7 / 128, -5 / 128, 1 / 128   # 2.5, 3.5, -2.5, 0.5 after scaling
    x[6] = 0.75 / 64
    d, s, q, bs = q8k_fields(O.quantize_q8_K(x), 1)
    assert d[0] == np.float32(1.0 / 64.0)
    assert list(q[0, :7]) == [-127, 127, 2, 4, -2, 0, 1]       # ties to even: 2.5->2, 3.5->4, -2.5->-2, 0.5->0
    assert (q[0, 7:] == 0).all()
    assert (bs[0] == q[0].reshape(16, 16).sum(1)).all()
    assert s[0] == np.float32(d[0] * np.float32(q[0].sum()))
    # the positive value first: it sets the scale and maps to -127
    x[0], x[1] = -m, m
    d, _, q, _ = q8k_fields(O.quantize_q8_K(x), 1)
    assert d[0] == np.float32(-1.0 / 64.0) and q[0, 0] == -127 and q[0, 1] == 127 and q[0, 2] == -2


def test_q8K_zero_block():
    assert (O.quantize_q8_K(np.zeros(512, np.float32)) == 0).all()


@pytest.mark.parametrize("seed", [0, 1])
def test_q8K_invariants_random(seed):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.normal(0, 1, 256 * 6), rng.standard_t(2, 256 * 2) * 1e-3]).astype(np.float32)
    x[256 * 3:256 * 3 + 100] = 0
    nb = x.size // 256
    d, _, q, bs = q8k_fields(O.quantize_q8_K(x), nb)
    X = x.reshape(nb, 256).astype(np.float64)
    for b in range(nb):
        j = int(np.argmax(np.abs(X[b])))                 # first index of the largest magnitude
        assert q[b, j] == -127
        err = np.abs(X[b] - d[b] * q[b])
        assert (err <= abs(d[b]) * (0.5 + 1e-6)).all()
        assert abs(d[b] * -127 - X[b, j]) <= abs(X[b, j]) * 2 * EPS
    assert (bs == q.reshape(nb, 16, 16).sum(2)).all()


# ---------------------------------------------------------- IQ3_S x Q8_K pins

def _isums(w_row, q, nb):
    lv, _ = npref.levels(O.IQ3_S, w_row, nb * 256)      # signed level * multiplier, int64
    return (lv.reshape(nb, 256) * q).sum(1)


def _dw(w_row, nb):
    B = np.asarray(w_row, np.uint8).reshape(nb, 110)
    return npref.f16(B[:, 0].astype(np.uint16) | (B[:, 1].astype(np.uint16) << 8))


@pytest.mark.parametrize("seed", range(4))
def test_vec_dot_single_superblock_exact(seed):
    rng = np.random.default_rng(seed)
    w = O.quantize(O.IQ3_S, rng.normal(0, 0.05, 256).astype(np.float32))
    y = O.quantize_q8_K(rng.normal(0, 1, 256).astype(np.float32))
    d, _, q, _ = q8k_fields(y, 1)
    isum = _isums(w, q, 1)[0]
    want = np.float32(np.float32(_dw(w, 1)[0] * d[0]) * np.float32(isum))
    assert O.vec_dot_iq3s_q8K(w, y, 256) == want
    assert cpu.vec_dot_iq3s_q8K(256, w, y) == want


def test_vec_dot_many_superblocks_bound():
    rng = np.random.default_rng(7)
    n = 256 * 16
    w = O.quantize(O.IQ3_S, rng.normal(0, 0.05, n).astype(np.float32))
    y = O.quantize_q8_K(rng.normal(0, 1, n).astype(np.float32))
    d, _, q, _ = q8k_fields(y, 16)
    terms = _dw(w, 16).astype(np.float64) * d * _isums(w, q, 16)
    got = O.vec_dot_iq3s_q8K(w, y, n)
    assert abs(got - terms.sum()) <= 4 * 16 * EPS * np.abs(terms).sum()
    assert cpu.vec_dot_iq3s_q8K(n, w, y) == got


def test_gemv_tracks_float_product():
    rng = np.random.default_rng(3)
    R, Cn = 64, 1024
    W = O.quantize(O.IQ3_S, rng.normal(0, 0.05, R * Cn).astype(np.float32))
    x = rng.normal(0, 1, Cn).astype(np.float32)
    y = O.gemv_iq3s_q8K(W, x, R, Cn)
    Wd = npref.dequant(O.IQ3_S, W, Cn)
    d, _, _, _ = q8k_fields(O.quantize_q8_K(x), Cn // 256)
    bound = (np.abs(Wd).reshape(R, -1, 256).sum(2) * np.abs(d) * 0.5).sum(1) * (1 + 1e-3) + 1e-6
    assert (np.abs(y - Wd @ x.astype(np.float64)) <= bound).all()


# ------------------------------------------------------------ expert loop pins

H, F, E = 512, 256, 6


@pytest.fixture(scope="module")
def bank():
    rng = np.random.default_rng(11)
    return iq3s_bank(rng, E, F, H), iq3s_bank(rng, E, F, H), iq3s_bank(rng, E, H, F)


def test_ncmoe_single_expert_composition(bank):
    g, u, d = bank
    x = np.random.default_rng(1).normal(0, 1, H).astype(np.float32)
    gg = O.gemv_iq3s_q8K(g[4], x, F, H)
    uu = O.gemv_iq3s_q8K(u[4], x, F, H)
    h = (gg / (np.float32(1) + np.exp(-gg))) * uu                   # float32 throughout, as moe_ffn.rs:1566-1570
    want = O.gemv_iq3s_q8K(d[4], h.astype(np.float32), H, F)
    got = O.ncmoe(x, g, u, d, [4], [1.0], H, F)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()   # numpy's exp vs libm's expf
    assert (cpu.iq3s_swiglu_expert_cpu(g[4], u[4], d[4], x, F, H) == got).all()


def test_ncmoe_weighted_sum_order(bank):
    g, u, d = bank
    x = np.random.default_rng(2).normal(0, 1, H).astype(np.float32)
    ids, wts = [1, 3, 5], np.array([0.5, 0.25, 0.125], np.float32)
    parts = [O.ncmoe(x, g, u, d, [e], [1.0], H, F) for e in ids]
    acc = np.zeros(H, np.float32)
    for w, p in zip(wts, parts):
        acc = acc + w * p
    assert (O.ncmoe(x, g, u, d, ids, wts, H, F) == acc).all()


def test_ncmoe_vs_float64(bank):
    g, u, d = bank
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, H).astype(np.float32)
    ids = np.array([0, 2, 3, 5], np.int32)
    wts = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    ref = np.zeros(H)
    for e, w in zip(ids, wts):
        gg = npref.dequant(O.IQ3_S, g[e], H) @ x
        uu = npref.dequant(O.IQ3_S, u[e], H) @ x
        h = gg / (1 + np.exp(-gg)) * uu
        ref += w * (npref.dequant(O.IQ3_S, d[e], F) @ h)
    got = O.ncmoe(x, g, u, d, ids, wts, H, F)
    # two Q8_K roundings (x, then h): about 1/254 of each block's scale per value
    assert np.linalg.norm(got - ref) <= 0.03 * np.linalg.norm(ref)


# ------------------------------------------------------- product vs the oracle

def test_header_symbols_exported_and_bound():
    txt = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "chimere_cpu.h")).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b((?:ggml_ffi|chimere)_[a-z0-9_A-Z]+)\s*\(", txt)))
    assert len(names) == 8
    L = cpu.lib()
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == {s[0] for s in cpu.SIGNATURES}
    assert cpu.iq3s_row_bytes(2048) == 880 and L.ggml_ffi_q8k_row_bytes(2048) == 8 * 296


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q8K_product_equals_oracle(seed):
    rng = np.random.default_rng(seed)
    x = (rng.normal(0, 1, 256 * 9) * rng.choice([1e-4, 1, 300], 256 * 9)).astype(np.float32)
    x[256:512] = 0
    x[600] = -x[600:900].__abs__().max()
    assert (cpu.quantize_q8_K(x) == O.quantize_q8_K(x)).all()


@pytest.mark.parametrize("rows,cols,nt", [(1, 256, 1), (37, 768, 3), (512, 2048, 4), (96, 4096, 0)])
def test_gemv_product_equals_oracle(rows, cols, nt):
    rng = np.random.default_rng(rows + cols)
    W = O.quantize(O.IQ3_S, rng.normal(0, 0.03, rows * cols).astype(np.float32))
    x = rng.normal(0, 1, cols).astype(np.float32)
    want = O.gemv_iq3s_q8K(W, x, rows, cols)
    assert (cpu.iq3s_gemv_cpu_parallel(W, x, rows, cols, nt).view(np.uint32) == want.view(np.uint32)).all()
    assert (cpu.iq3s_gemv_cpu(W, x, rows, cols).view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("ids,nt", [([0], 1), ([5, 1, 3, 0, 2, 4, 1, 5], 4), ([2, 2, 2], 0), ([3, 0], 7)])
def test_ncmoe_product_equals_oracle(bank, ids, nt):
    g, u, d = bank
    rng = np.random.default_rng(len(ids) + nt)
    x = rng.normal(0, 1, H).astype(np.float32)
    w = rng.random(len(ids)).astype(np.float32)
    w /= w.sum()
    want = O.ncmoe(x, g, u, d, ids, w, H, F)
    got = cpu.ncmoe_experts(g, u, d, ids, w, x, H, F, nthreads=nt)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


def test_ncmoe_zero_hidden_and_zero_weight(bank):
    g, u, d = bank
    z = cpu.ncmoe_experts(g, u, d, [1, 2], [0.5, 0.5], np.zeros(H, np.float32), H, F)
    assert (z == 0).all()
    x = np.random.default_rng(9).normal(0, 1, H).astype(np.float32)
    a = cpu.ncmoe_experts(g, u, d, [1, 2], [1.0, 0.0], x, H, F)
    assert (a == cpu.ncmoe_experts(g, u, d, [1], [1.0], x, H, F)).all()


def test_ncmoe_rejects_bad_arguments(bank):
    g, u, d = bank
    x = np.zeros(H, np.float32)
    with pytest.raises(ValueError):
        cpu.ncmoe_experts(g, u, d, [E], [1.0], x, H, F)             # expert id out of range
    with pytest.raises(ValueError):
        cpu.ncmoe_experts(g, u, d, [-1], [1.0], x, H, F)
    with pytest.raises(ValueError):
        cpu.ncmoe_experts(g, u, d, [0], [1.0], x, H + 256, F)       # slices too small for the shape
    with pytest.raises(ValueError):
        cpu.ncmoe_experts(g, u, d, [0], [1.0], x, H, 200)           # not a multiple of 256
    with pytest.raises(ValueError):
        cpu.iq3s_gemv_cpu(g[0], x, F, 300)


@pytest.mark.parametrize("env,isa", [({"CHIMERE_CPU_PORTABLE": "1"}, 0), ({"CHIMERE_CPU_NO_AVX512": "1"}, 1)])
def test_other_integer_kernels_equal_the_oracle(env, isa):
    """The AVX2 and portable integer loops (chosen where AVX-512 / AVX2 are
    missing) give the same bits as the oracle."""
    if isa == 1 and not open("/proc/cpuinfo").read().count(" avx2"):
        pytest.skip("no AVX2 on this host")
    code = ("import sys, numpy as np; sys.path[:0] = [%r, %r]; import oracle as O; from chimere_amd import cpu;"
            "rng = np.random.default_rng(4); W = O.quantize(O.IQ3_S, rng.normal(0, .03, 40 * 1024).astype(np.float32));"
            "x = rng.normal(0, 1, 1024).astype(np.float32);"
            "assert cpu.lib().chimere_cpu_isa() == %d, cpu.lib().chimere_cpu_isa();"
            "y = cpu.iq3s_gemv_cpu(W, x, 40, 1024); w = O.gemv_iq3s_q8K(W, x, 40, 1024);"
            "assert (y.view(np.uint32) == w.view(np.uint32)).all(); print('ok')") % (ROOT, os.path.join(ROOT, "tests"), isa)
    r = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, **env), capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr


def test_isa_in_use():
    flags = open("/proc/cpuinfo").read()
    want = 2 if (" avx512f" in flags and " avx512bw" in flags) else 1 if " avx2" in flags else 0
    assert cpu.lib().chimere_cpu_isa() == want


def test_q8k_minus_128_same_on_every_isa():
    """A caller-supplied Q8_K block holding -128 (which the library's
    quantizer never emits): the portable, AVX2 and AVX-512 integer loops give
    the same bits (negation under a sign bit wraps in every one of them)."""
    code = ("import sys, numpy as np; sys.path[:0] = [%r]; from chimere_amd import cpu;"
            "rng = np.random.default_rng(11); w = rng.integers(0, 256, 2 * 110, dtype=np.uint8);"
            "w[0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8); w[110:112] = w[0:2];"
            "y = np.zeros(2 * 296, np.uint8); q = rng.integers(-128, 128, 512).astype(np.int8);"
            "q[::7] = -128; y[8:264] = q[:256].view(np.uint8); y[296 + 8:296 + 264] = q[256:].view(np.uint8);"
            "y[0:4] = np.frombuffer(np.float32(0.02).tobytes(), np.uint8); y[296:300] = y[0:4];"
            "print(repr(np.float32(cpu.vec_dot_iq3s_q8K(512, w, y)).view(np.uint32)))") % ROOT
    out = set()
    for env in ({"CHIMERE_CPU_PORTABLE": "1"}, {"CHIMERE_CPU_NO_AVX512": "1"}, {}):
        r = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, **env), capture_output=True, text=True,
                           timeout=120)
        assert r.returncode == 0, r.stderr
        out.add(r.stdout.strip())
    assert len(out) == 1, out
