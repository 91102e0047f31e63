"""GPU parity of the activation quantizer, weight quantizers and block-quantized
GEMV entry points against the CPU oracle, through the C ABI.

Bar: Q8_1 bytes, weight bytes and int32 block dots bit-exact; fp32 GEMV
outputs bit-exact against the oracle run in the kernels' documented order
(L=16 lanes, G=1) -- stronger than the required max relative error of 1e-5
(Q8_0/Q4_0) / 1e-4 (IQ3_S) normalised by ||y||, which is asserted as well
against the order-free float64 result."""
import numpy as np
import pytest
import torch

import oracle as O
import npref
from chimere_amd import ggml_gpu as G

pytestmark = pytest.mark.gpu
TOL = {O.Q8_0: 1e-5, O.Q4_0: 1e-5, O.IQ3_S: 1e-4}


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("ncols,pad,batch", [(2048, 2048, 1), (512, 512, 8), (2000, 2048, 3), (4096, 4096, 2)])
def test_quantize_q8_1_bit_exact(dev, ncols, pad, batch):
    rng = np.random.default_rng(ncols + batch)
    x = rng.standard_normal((batch, ncols)).astype(np.float32) * np.float32(3)
    x[0, :32] = 0                                   # all-zero block
    x[-1, 40:72] = np.float32(2.0 ** 20)            # large, uniform block
    out = torch.zeros(batch, pad // 32 * 36, dtype=torch.uint8, device=dev)
    G.lib().chimere_quantize_q8_1_batched(G._ptr(dev_t(x, dev)), G._ptr(out), ncols, pad, batch, G._stream())
    G.check()
    ref = O.quantize_q8_1(x, pad)
    assert (host(out) == ref).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.IQ3_S])
def test_weight_quantizers_bit_exact(dev, t):
    rng = np.random.default_rng(50 + t)
    x = rng.normal(0, 0.02, (64, 2048)).astype(np.float32)
    x[3, :256] = 0                                   # zero super-block
    x[5, :256] *= 1e4
    out = torch.zeros(64 * O.row_bytes(t, 2048), dtype=torch.uint8, device=dev)
    G.quantize_weights(t, dev_t(x, dev), out)
    assert (host(out) == O.quantize(t, x).reshape(-1)).all()


def _case(t, nrows, ncols, seed):
    rng = np.random.default_rng(seed)
    w = O.quantize(t, rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32))
    x = rng.standard_normal(ncols).astype(np.float32)
    return w, x, O.quantize_q8_1(x)


SHAPES = [(4096, 2048), (37, 2048), (512, 2048), (2048, 512), (300, 8192), (16, 256), (256, 4096)]


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.IQ3_S])
@pytest.mark.parametrize("nrows,ncols", SHAPES)
def test_gemv_bit_exact(dev, t, nrows, ncols):
    print(f"gemv type={t} {nrows}x{ncols}", flush=True)
    w, x, xq = _case(t, nrows, ncols, nrows * 7 + ncols + t)
    wd, xd, xqd = dev_t(w, dev), dev_t(x, dev), dev_t(xq, dev)
    y = torch.zeros(nrows, dtype=torch.float32, device=dev)
    {O.Q8_0: G.ggml_gpu_gemv_q8_0_q8, O.Q4_0: G.ggml_gpu_gemv_q4_0_q8, O.IQ3_S: G.ggml_gpu_gemv_iq3s_q8}[t](
        wd, xqd, y, nrows, ncols)
    yg = host(y)
    yo = O.gemv(t, w, xq, ncols, nrows, L=16, G=1)
    assert (yg.view(np.uint32) == yo.view(np.uint32)).all()
    y64 = npref.gemv_f64(t, w, xq, ncols)
    assert np.linalg.norm(yg - y64) / np.linalg.norm(y64) < TOL[t]
    # block dots (debug entry point): exact int32
    bd = torch.zeros(nrows, ncols // 32, dtype=torch.int32, device=dev)
    G.block_dots(t, wd, xqd, bd, nrows, ncols)
    assert (host(bd) == O.block_dots(t, w, xq, ncols, nrows)).all()
    # fused f32 -> Q8_1 -> GEMV entry point, scratch padded to 512
    scratch = torch.zeros(G.q8_1_row_bytes(ncols), dtype=torch.uint8, device=dev)
    y2 = torch.zeros(nrows, dtype=torch.float32, device=dev)
    {O.Q8_0: G.ggml_gpu_gemv_q8_0_f32, O.Q4_0: G.ggml_gpu_gemv_q4_0_f32, O.IQ3_S: G.ggml_gpu_gemv_iq3s_f32}[t](
        wd, xd, y2, scratch, nrows, ncols)
    assert (host(y2).view(np.uint32) == yo.view(np.uint32)).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.IQ3_S])
@pytest.mark.parametrize("H", [1024, 2048])
def test_gemv_batched_by_expert_ids(dev, t, H):
    """ggml_gpu_cuda.cu:243-279 semantics: slot k uses expert ids[k] and input
    k*input_stride (0 = shared).  H=2048: whole 64-block chunks (the GEMV's
    compile-time chunk path); H=1024: a partial chunk."""
    rng = np.random.default_rng(70 + t)
    E, F, K = 12, 64, 5
    w = O.quantize(t, rng.normal(0, 0.02, (E * F, H)).astype(np.float32)).reshape(E, -1)
    xs = rng.standard_normal((K, H)).astype(np.float32)
    xq = O.quantize_q8_1(xs)                        # [K, row bytes]
    ids = np.array([7, 0, 11, 7, 3], np.int32)
    fn = {O.Q8_0: G.ggml_gpu_gemv_q8_0_batched, O.Q4_0: G.ggml_gpu_gemv_q4_0_batched,
          O.IQ3_S: G.ggml_gpu_gemv_iq3s_batched}[t]
    wd, xqd, idd = dev_t(w, dev), dev_t(xq, dev), dev_t(ids, dev)
    for stride in (0, xq.shape[1]):
        y = torch.zeros(K * F, dtype=torch.float32, device=dev)
        fn(wd, xqd, y, idd, F, H, w.shape[1], stride, K)
        yg = host(y).reshape(K, F)
        for k in range(K):
            xk = xq[k] if stride else xq[0]
            yo = O.gemv(t, w[ids[k]], xk, H, F)
            assert (yg[k].view(np.uint32) == yo.view(np.uint32)).all()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.IQ3_S])
@pytest.mark.parametrize("ntok", [1, 2, 5, 8])
def test_gemv_multi_token(dev, t, ntok):
    rng = np.random.default_rng(90 + t * 10 + ntok)
    nrows, ncols = 200, 2048
    w = O.quantize(t, rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32))
    xq = O.quantize_q8_1(rng.standard_normal((ntok, ncols)).astype(np.float32))
    y = torch.zeros(ntok, nrows, dtype=torch.float32, device=dev)
    G.gemv_multi(t, dev_t(w, dev), dev_t(xq, dev), y, nrows, ncols, ntok)
    yo = O.gemv(t, w, xq, ncols, nrows, ntok=ntok, xq_stride=xq.shape[1])
    assert (host(y).reshape(ntok, nrows).view(np.uint32) == np.asarray(yo).reshape(ntok, nrows).view(np.uint32)).all()
    # the per-type entry point gives the same bits
    import ctypes as C
    from chimere_amd._lib import check, lib
    fn = {O.Q4_0: "chimere_mmvq_q4_0_multi", O.Q8_0: "chimere_mmvq_q8_0_multi", O.IQ3_S: "chimere_mmvq_iq3s_multi"}[t]
    y2 = torch.zeros_like(y)
    wd, xd = dev_t(w, dev), dev_t(xq, dev)
    getattr(lib(), fn)(C.c_void_p(wd.data_ptr()), C.c_void_p(xd.data_ptr()), C.c_void_p(y2.data_ptr()), ncols, nrows,
                       xq.shape[1] // 36, ntok, G._stream())
    check()
    assert (host(y2).view(np.uint32) == host(y).view(np.uint32)).all()


def test_gemv_synth251_fixture(dev):
    """The reference's synthetic IQ3_S bytes (fused_gate_up.rs:386-412): block
    dots equal the committed golden file."""
    import os
    W = (np.arange(16 * 8 * 110) % 251).astype(np.uint8)
    xq = np.zeros(64 * 36, np.uint8)
    for b in range(64):
        xq[b * 36 + 1] = 0x10
        xq[b * 36 + 4:b * 36 + 36] = np.arange(32) % 5
    bd = torch.zeros(16, 64, dtype=torch.int32, device=dev)
    G.block_dots(O.IQ3_S, dev_t(W, dev), dev_t(xq, dev), bd, 16, 2048)
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "iq3s_synth251_block_dots.npy"))
    assert (host(bd) == gold).all()


def test_q4_0_head_full_size(dev):
    """Config 2 at full size (151936 x 2048 Q4_0, 175 MB): weights drawn and
    quantized on the device, GEMV checked bit-exact against the oracle on the
    same bytes, plus the linearity property y(-x) = -y(x)."""
    V, H = 151936, 2048
    g = torch.Generator(device=dev).manual_seed(2)
    wf = torch.randn(V, H, generator=g, device=dev) * 0.02
    w = torch.empty(V * H // 32 * 18, dtype=torch.uint8, device=dev)
    G.quantize_weights(O.Q4_0, wf, w)
    del wf
    x = torch.randn(H, generator=g, device=dev)
    xq = torch.zeros(G.q8_1_row_bytes(H), dtype=torch.uint8, device=dev)
    G.ggml_gpu_quantize_q8_1(x, xq, H)
    y = torch.zeros(V, dtype=torch.float32, device=dev)
    G.ggml_gpu_gemv_q4_0_q8(w, xq, y, V, H)
    yo = O.gemv(O.Q4_0, host(w), host(xq), H, V)
    yg = host(y)
    assert (yg.view(np.uint32) == yo.view(np.uint32)).all()
    G.ggml_gpu_quantize_q8_1(-x, xq, H)
    G.ggml_gpu_gemv_q4_0_q8(w, xq, y, V, H)
    assert (host(y) == -yg).all()


# ---- ggml K-quants and MXFP4 (ffi/ggml_cuda_gemv.cu:118-175, 292-460)

KQ_FN = {O.Q4_K: ("chimere_mmvq_q4k", "chimere_mmvq_q4k_f32"), O.Q5_K: ("chimere_mmvq_q5k", "chimere_mmvq_q5k_f32"),
         O.Q6_K: ("chimere_mmvq_q6k", "chimere_mmvq_q6k_f32"), O.MXFP4: ("chimere_mmvq_mxfp4", None)}
KQ_SHAPES = [(4096, 2048), (37, 2304), (300, 4096), (16, 256), (512, 4096)]


@pytest.mark.parametrize("t,nrows,ncols", [(t, r, c) for r, c in KQ_SHAPES for t in (O.Q4_K, O.Q5_K, O.Q6_K, O.MXFP4)]
                         + [(O.MXFP4, 64, 2080), (O.MXFP4, 19, 96)])
def test_kquant_gemv_bit_exact(dev, t, nrows, ncols):
    """Bit-exact against the oracle's (L=16, G=1) order; within 1e-5 of the
    float64 result; int32 block dots exact; the fused f32 entry gives the same
    bits.  (64, 2080) and (19, 96) are MXFP4-only shapes (rows not 4-byte
    aligned)."""
    print(f"kquant gemv type={t} {nrows}x{ncols}", flush=True)
    rng = np.random.default_rng(nrows * 3 + ncols + t)
    w = npref.rand_kq(t, nrows, ncols, rng)
    x = rng.standard_normal(ncols).astype(np.float32)
    pad = G.pad(ncols, 512)
    xq = O.quantize_q8_1(x, pad)
    wd, xd, xqd = dev_t(w, dev), dev_t(x, dev), dev_t(xq, dev)
    import ctypes as C
    from chimere_amd._lib import check, lib
    y = torch.zeros(nrows, dtype=torch.float32, device=dev)
    q8, f32 = KQ_FN[t]
    getattr(lib(), q8)(C.c_void_p(wd.data_ptr()), C.c_void_p(xqd.data_ptr()), C.c_void_p(y.data_ptr()), ncols,
                       nrows, pad // 32, G._stream())
    check()
    yg = host(y)
    yo = O.gemv(t, w, xq, ncols, nrows, L=16, G=1)
    assert (yg.view(np.uint32) == yo.view(np.uint32)).all()
    y64 = npref.kq_gemv_f64(t, w, xq, ncols)
    assert np.linalg.norm(yg - y64) / np.linalg.norm(y64) < 1e-5
    bd = torch.zeros(nrows, ncols // 32, dtype=torch.int32, device=dev)
    G.block_dots(t, wd, xqd, bd, nrows, ncols)
    assert (host(bd) == O.block_dots(t, w, xq, ncols, nrows)).all()
    scratch = torch.zeros(pad // 32 * 36, dtype=torch.uint8, device=dev)
    y2 = torch.zeros(nrows, dtype=torch.float32, device=dev)
    {O.Q4_K: G.ggml_gpu_gemv_q4k_f32, O.Q5_K: G.ggml_gpu_gemv_q5k_f32, O.Q6_K: G.ggml_gpu_gemv_q6k_f32,
     O.MXFP4: G.ggml_gpu_gemv_mxfp4_f32}[t](wd, xd, y2, scratch, nrows, ncols)
    assert (host(y2).view(np.uint32) == yo.view(np.uint32)).all()


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.MXFP4])
def test_kquant_multi_token(dev, t):
    rng = np.random.default_rng(400 + t)
    nrows, ncols, ntok = 100, 2048, 3
    w = npref.rand_kq(t, nrows, ncols, rng)
    xq = O.quantize_q8_1(rng.standard_normal((ntok, ncols)).astype(np.float32))
    y = torch.zeros(ntok, nrows, dtype=torch.float32, device=dev)
    G.gemv_multi(t, dev_t(w, dev), dev_t(xq, dev), y, nrows, ncols, ntok)
    yo = O.gemv(t, w, xq, ncols, nrows, ntok=ntok, xq_stride=xq.shape[1])
    assert (host(y).view(np.uint32) == np.asarray(yo).view(np.uint32)).all()


def test_mxfp4_batched_device_ids(dev):
    """chimere_mmvq_mxfp4_batched reads the expert ids on the device (the
    reference's host-side dereference, ggml_cuda_gemv.cu:438-444, is not kept)."""
    rng = np.random.default_rng(39)
    E, F, H, K = 6, 48, 1024, 4
    w = npref.rand_kq(O.MXFP4, E * F, H, rng).reshape(E, -1)
    xq = O.quantize_q8_1(rng.standard_normal((K, H)).astype(np.float32))
    ids = np.array([5, 0, 5, 2], np.int32)
    wd, xqd, idd = dev_t(w, dev), dev_t(xq, dev), dev_t(ids, dev)
    for stride in (0, xq.shape[1]):
        y = torch.zeros(K * F, dtype=torch.float32, device=dev)
        G.ggml_gpu_gemv_mxfp4_batched(wd, xqd, y, idd, F, H, w.shape[1], stride, K)
        yg = host(y).reshape(K, F)
        for k in range(K):
            yo = O.gemv(O.MXFP4, w[ids[k]], xq[k] if stride else xq[0], H, F)
            assert (yg[k].view(np.uint32) == yo.view(np.uint32)).all()


@pytest.mark.parametrize("nrows,ncols", [(4096, 2048), (37, 2048), (2048, 512), (300, 8192)])
def test_gemv_q4_0_sform_bit_exact(dev, nrows, ncols):
    """ggml's s-form Q4_0 block term (chimere_mmvq_q4_0_sform) against the
    oracle's restatement, bit for bit; and within the bound of the exact form."""
    print(f"gemv q4_0 s-form {nrows}x{ncols}", flush=True)
    w, x, xq = _case(O.Q4_0, nrows, ncols, nrows * 11 + ncols)
    wd, xqd = dev_t(w, dev), dev_t(xq, dev)
    ys = torch.zeros(nrows, dtype=torch.float32, device=dev)
    ye = torch.zeros(nrows, dtype=torch.float32, device=dev)
    G.ggml_gpu_gemv_q4_0_sform_q8(wd, xqd, ys, nrows, ncols)
    G.ggml_gpu_gemv_q4_0_q8(wd, xqd, ye, nrows, ncols)
    gs, ge = host(ys), host(ye)
    assert (gs.view(np.uint32) == O.gemv(O.Q4_0_SFORM, w, xq, ncols, nrows).view(np.uint32)).all()
    assert (ge.view(np.uint32) == O.gemv(O.Q4_0, w, xq, ncols, nrows).view(np.uint32)).all()
    # the forms differ by at most sum_b 8 |d_w| |s_x - d_x * sum(q_x)| per row (+ fp32 rounding)
    nb = ncols // 32
    xb = xq[:nb * 36].reshape(nb, 36)
    f16 = lambda b: np.frombuffer(np.ascontiguousarray(b).tobytes(), np.float16).astype(np.float64)  # noqa: E731
    dx, sx = f16(xb[:, 0:2]), f16(xb[:, 2:4])
    sq = xb[:, 4:].view(np.int8).astype(np.int64).sum(axis=1)
    dw = f16(w.reshape(nrows, nb, 18)[:, :, :2]).reshape(nrows, nb)
    bound = (8 * np.abs(dw) * np.abs(sx - dx * sq)[None, :]).sum(axis=1)
    diff = np.abs(gs.astype(np.float64) - ge)
    assert (diff <= bound + 1e-5 * np.abs(ge).max()).all() and diff.max() > 0
