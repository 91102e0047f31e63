"""GPU parity of the prefill MoE chunk (chimere_moe_prefill: int8 matrix-core
grouped GEMMs) against the CPU oracle, through the C ABI.

Bar: routing indices and weights bit-exact; per-token outputs bit-exact
against the oracle in the prefill order (L=1: one accumulator per row,
blocks in ascending order).  BASELINE config 5 (512 tokens, Q4_0, full
shape) is checked token by token against the oracle for the whole chunk,
plus chunk-independence and agreement with the decode entry point's
routing."""
import numpy as np
import pytest
import torch

import oracle as O
from chimere_amd.moe import MoeLayer
from test_gpu_moe import build, check_margin, host, oracle_run, qmat

pytestmark = pytest.mark.gpu


def prefill_check(layer, x, sample=None, margin=True):
    T = x.shape[0]
    if margin:
        check_margin(layer, x if sample is None else x[sample])
    ids = torch.full((T, layer.K), -1, dtype=torch.int32, device=x.device)
    wts = torch.zeros(T, layer.K, dtype=torch.float32, device=x.device)
    out = layer.prefill(x, ids=ids, wts=wts)
    og, ig, wg = host(out), host(ids), host(wts)
    rows = np.arange(T) if sample is None else np.asarray(sample)
    oo, io, wo = oracle_run(layer, x[rows], L=1)
    assert (ig[rows] == io).all(), "routing indices differ"
    assert (wg[rows].view(np.uint32) == wo.view(np.uint32)).all(), "routing weights differ"
    bad = np.nonzero((og[rows].view(np.uint32) != oo.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, f"tokens {rows[bad][:8]} differ, max |d| {np.abs(og[rows] - oo).max()}"
    return og, ig, wg


@pytest.mark.parametrize("et,st,gate_vec,K,E,T", [
    (O.Q4_0, O.Q4_0, False, 8, 64, 1),
    (O.Q4_0, O.Q4_0, True, 8, 64, 37),
    (O.Q8_0, O.Q8_0, True, 4, 16, 70),      # many pairs per expert: several tiles each
    (O.Q4_0, O.Q8_0, False, 2, 32, 5),
    (O.Q8_0, O.Q4_0, True, 8, 8, 9),        # K == E
    (O.Q4_0, None, False, 1, 4, 33),        # no shared expert, top-1
    (O.IQ3_S, O.IQ3_S, True, 8, 64, 37),    # IQ3_S: one superblock per K chunk, unaligned staging
    (O.IQ3_S, O.Q8_0, False, 4, 16, 70),    # the IQ3_S model layers' Q8_0 shared expert
    (O.IQ3_S, O.Q4_0, True, 8, 8, 9),
    (O.Q4_0, O.IQ3_S, False, 2, 32, 5),
])
def test_prefill_small(dev, et, st, gate_vec, K, E, T):
    print(f"prefill et={et} st={st} gate={gate_vec} K={K} E={E} T={T}", flush=True)
    layer = build(dev, 200 + K + E + T, H=1024, F=256, E=E, K=K, et=et, st=st, gate_vec=gate_vec)
    g = torch.Generator(device=dev).manual_seed(T)
    prefill_check(layer, torch.randn(T, 1024, generator=g, device=dev))


@pytest.mark.parametrize("et,st,gate_vec", [
    (O.IQ3_S, O.IQ3_S, True),
    (O.IQ3_S, O.Q4_0, False),
    (O.Q4_0, O.IQ3_S, True),
])
def test_prefill_aligned_rows(dev, et, st, gate_vec):
    """H = 2048: 880-byte IQ3_S rows are 16-byte aligned, so the gate/up GEMM
    runs the two-stage aligned-span path; 37 tokens leave partially filled
    16-pair tiles."""
    print(f"prefill aligned et={et} st={st} gate={gate_vec}", flush=True)
    layer = build(dev, 400 + et + st, H=2048, F=512, E=64, K=8, et=et, st=st, gate_vec=gate_vec)
    g = torch.Generator(device=dev).manual_seed(37)
    prefill_check(layer, torch.randn(37, 2048, generator=g, device=dev))


@pytest.mark.parametrize("et,st", [(O.IQ3_S, O.IQ3_S), (O.IQ3_S, O.Q8_0)])
def test_prefill_iq3s_down_spans(dev, et, st):
    """F = 1024: 440-byte IQ3_S down rows, four one-superblock K chunks per
    row; each row chunk starts at (440 r + 110 c) % 16 = 0, 2, ..., 14 bytes
    past a 16-byte boundary, so the down's per-row 16-byte span copies place
    it at every even offset of its LDS row (H = 512: the gate/up's 220-byte
    rows, not 16-byte aligned, take the one-stage path's row staging)."""
    print(f"prefill iq3s down spans et={et} st={st}", flush=True)
    layer = build(dev, 500 + et + st, H=512, F=1024, E=32, K=4, et=et, st=st, gate_vec=True)
    g = torch.Generator(device=dev).manual_seed(41)
    prefill_check(layer, torch.randn(41, 512, generator=g, device=dev))


def test_prefill_config5_512(dev):
    """512 tokens, H=2048, F=512, E=256, top-8, Q4_0 experts + Q4_0 shared:
    every token's output, index and weight bit-exact against the oracle.  All
    256 experts are selected, so every expert's tiles -- the 16-pair tiles of
    its tokens and its partly filled last tile -- are held to the oracle's
    bits."""
    layer = build(dev, 5)
    g = torch.Generator(device=dev).manual_seed(55)
    x = torch.randn(512, 2048, generator=g, device=dev)
    check_margin(layer, x, "config 5")
    og, ig, wg = prefill_check(layer, x, margin=False)
    assert np.isfinite(og).all()
    counts = np.bincount(ig.reshape(-1), minlength=256)
    assert (counts > 0).all(), "an expert is unused: its tiles would go unchecked"
    assert (counts % 16 != 0).any()         # partly filled last tiles occur
    # routing of every token equals the decode entry point's, bit for bit
    for t0 in range(0, 512, 8):
        ids = torch.zeros(8, 8, dtype=torch.int32, device=dev)
        wts = torch.zeros(8, 8, dtype=torch.float32, device=dev)
        layer.forward(x[t0:t0 + 8], ids=ids, wts=wts)
        assert (host(ids) == ig[t0:t0 + 8]).all()
        assert (host(wts).view(np.uint32) == wg[t0:t0 + 8].view(np.uint32)).all()
    # chunk independence: a token's output does not depend on the rest of the chunk
    part = host(layer.prefill(x[100:160].contiguous()))
    assert (part.view(np.uint32) == og[100:160].view(np.uint32)).all()
    # and against the decode path (L=16 order) only the fp32 order differs
    dec = host(layer.forward(x[:8]))
    for m in range(8):
        assert np.linalg.norm(dec[m] - og[m]) <= 2e-3 * np.linalg.norm(og[m])


def test_prefill_iq3s_full_shape(dev):
    """IQ3_S experts at the model's shape (H=2048, F=512, E=256, top-8) with the
    Q8_0 shared expert, 96 tokens, uniform and Zipf(1.1) routing: every token
    against the oracle."""
    for zipf in (False, True):
        layer = build(dev, 31 + zipf, et=O.IQ3_S, st=O.Q8_0, zipf=zipf)
        g = torch.Generator(device=dev).manual_seed(77)
        prefill_check(layer, torch.randn(96, 2048, generator=g, device=dev))


def test_prefill_repeat_and_zero(dev):
    layer = build(dev, 12, H=1024, F=256, E=32, K=4)
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(40, 1024, generator=g, device=dev)
    first = host(layer.prefill(x))
    for T in (3, 40, 17):
        assert (host(layer.prefill(x[:T].contiguous())) == first[:T]).all()
    z = host(layer.prefill(torch.zeros(4, 1024, device=dev)))
    assert np.isfinite(z).all()


def test_prefill_more_pairs_than_plan_threads(dev):
    """T * K above 4096: the plan's count and scatter passes take several
    batches of pairs.  Sampled tokens bit-exact against the oracle, every
    routing index against the decode entry point's, and the first tokens
    equal to a shorter chunk's (each token's output depends only on it)."""
    layer = build(dev, 31, H=1024, F=256, E=64, K=8)
    g = torch.Generator(device=dev).manual_seed(17)
    T = 700                                     # 5600 pairs
    x = torch.randn(T, 1024, generator=g, device=dev)
    sample = list(range(0, T, 37)) + [T - 1]
    og, ig, wg = prefill_check(layer, x, sample=sample)
    short = host(layer.prefill(x[:130].contiguous()))
    assert (short == og[:130]).all()
    ids = torch.zeros(8, layer.K, dtype=torch.int32, device=dev)
    wts = torch.zeros(8, layer.K, dtype=torch.float32, device=dev)
    for t0 in (0, 350, 692):
        layer.forward(x[t0:t0 + 8].contiguous(), ids=ids, wts=wts)
        assert (host(ids) == ig[t0:t0 + 8]).all()


def test_prefill_unaligned_output(dev):
    """An output buffer that is not 16-byte aligned (a view one float into an
    allocation) gets the same bits as an aligned one."""
    layer = build(dev, 13, H=1024, F=256, E=32, K=4)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(9, 1024, generator=g, device=dev)
    want = host(layer.prefill(x))
    buf = torch.full((9 * 1024 + 1,), float("nan"), device=dev)
    out = buf[1:].view(9, 1024)
    layer.prefill(x, out=out)
    assert (host(out) == want).all()
    assert np.isnan(host(buf)[0])


def kq_layer(dev, seed, et, st, H, F, E, K, gate_vec=True):
    """Experts of type et (device quantizer), a K-quant shared expert of type
    st from the independent packer (valid random blocks)."""
    import npref
    g = torch.Generator(device=dev).manual_seed(seed)
    router = torch.randn(E, H, generator=g, device=dev) * 0.02
    gate, up, down = qmat(et, F, H, E, g, dev), qmat(et, F, H, E, g, dev), qmat(et, H, F, E, g, dev)
    rng = np.random.default_rng(seed)
    sh = tuple(torch.from_numpy(np.ascontiguousarray(npref.rand_kq(st, r, c, rng).reshape(-1))).to(dev)
               for r, c in ((F, H), (F, H), (H, F)))
    gw = torch.randn(H, generator=g, device=dev) * 0.02 if gate_vec else None
    return MoeLayer(router, gate, up, down, et, K, shared=sh, shared_type=st, sh_gate_w=gw)


@pytest.mark.parametrize("et,st,H,F,E,K,T", [
    (O.Q4_0, O.Q5_K, 1024, 256, 32, 4, 37),
    (O.Q8_0, O.Q4_K, 1024, 256, 16, 8, 20),
    (O.IQ3_S, O.Q5_K, 1024, 256, 64, 8, 9),
    (O.Q4_0, O.Q6_K, 1024, 256, 32, 4, 37),
    (O.Q8_0, O.Q6_K, 1024, 512, 16, 8, 20),
    (O.IQ3_S, O.Q6_K, 2048, 256, 64, 8, 9),
])
def test_prefill_kquant_shared_small(dev, et, st, H, F, E, K, T):
    """K-quant shared expert on the MFMA path (scale on the int32 result, the
    min term added per block), bit-exact against the oracle's L=1 order."""
    print(f"prefill kquant shared et={et} st={st} H={H} F={F} E={E} K={K} T={T}", flush=True)
    layer = kq_layer(dev, 800 + et + st + T, et, st, H, F, E, K)
    g = torch.Generator(device=dev).manual_seed(T)
    prefill_check(layer, torch.randn(T, H, generator=g, device=dev))


def test_prefill_q6k_shared_full_shape(dev):
    """A Q6_K shared expert (two int8 scales per 32-element block: the two
    16-element halves in separate products, combined exactly before the
    block's one rescale) at the model shape: 1680-byte gate/up rows on the
    two-stage path, 420-byte down rows on the one-stage path, every token
    bit-exact against the oracle's L=1 order."""
    print("prefill IQ3_S + Q6_K shared, full shape, 40 tokens", flush=True)
    layer = kq_layer(dev, 890, O.IQ3_S, O.Q6_K, 2048, 512, 256, 8)
    g = torch.Generator(device=dev).manual_seed(89)
    prefill_check(layer, torch.randn(40, 2048, generator=g, device=dev))


def test_prefill_model_layer_types_full_shape(dev):
    """The reference model's layer types at its shape: IQ3_S experts (H=2048,
    F=512, E=256, top-8) with the Q5_K shared expert and its sigmoid gate,
    96 tokens, every token bit-exact against the oracle."""
    print("prefill IQ3_S + Q5_K shared, full shape, 96 tokens", flush=True)
    layer = kq_layer(dev, 880, O.IQ3_S, O.Q5_K, 2048, 512, 256, 8)
    g = torch.Generator(device=dev).manual_seed(88)
    prefill_check(layer, torch.randn(96, 2048, generator=g, device=dev))
