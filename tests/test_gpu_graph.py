"""The fused MoE layer under HIP-graph capture (the reference runs it inside
a captured decode step: cs/src/cuda_graph.rs, compute_graph.rs:2020-2060).

A layer call is captured once with static input / output buffers, then the
graph is replayed several times with new inputs copied into the static input
and with eager layer calls (other inputs, other output buffers) and host
synchronisations between the replays.  Every replay must reproduce, bit for
bit, the eager call on the same input: the workspace's counters and flags
must return to their start state within each call, and nothing in a call may
depend on a value captured at capture time."""
import numpy as np
import pytest
import torch

import oracle as O
from chimere_amd.moe import MoeLayer
from test_gpu_moe import build, host, oracle_run, qmat

pytestmark = pytest.mark.gpu


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _check_replays(layer, call, M, H, K, dev, seed, order=16):
    gx = torch.Generator(device=dev).manual_seed(seed)
    inputs = [torch.randn(M, H, generator=gx, device=dev) for _ in range(3)]
    want = []
    for x in inputs:   # eager results
        ids = torch.empty(M, K, dtype=torch.int32, device=dev)
        wts = torch.empty(M, K, device=dev)
        out = call(layer, x, torch.empty_like(x), ids, wts)
        torch.cuda.synchronize()
        want.append((out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()))
    xs = torch.empty(M, H, device=dev)
    os_ = torch.full((M, H), float("nan"), device=dev)
    ids_s = torch.empty(M, K, dtype=torch.int32, device=dev)
    wts_s = torch.empty(M, K, device=dev)
    xs.copy_(inputs[0])
    g = _capture(lambda: call(layer, xs, os_, ids_s, wts_s))
    other = torch.randn(M, H, generator=gx, device=dev)
    for rep, i in enumerate([0, 1, 2, 1, 0, 2]):
        xs.copy_(inputs[i])
        os_.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = (os_.cpu().numpy(), ids_s.cpu().numpy(), wts_s.cpu().numpy())
        for name, a, b in zip(("out", "ids", "wts"), got, want[i]):
            assert np.array_equal(a, b), f"replay {rep} (input {i}): {name} differs from the eager call"
        if rep < 3:   # the first replay of each input against the oracle too
            oo, io, wo = oracle_run(layer, inputs[i], L=order)
            assert (got[1] == io).all() and (got[2].view(np.uint32) == wo.view(np.uint32)).all()
            assert (got[0].view(np.uint32) == oo.view(np.uint32)).all(), f"replay {rep}: output differs from the oracle"
        call(layer, other, torch.empty_like(other), None, None)   # eager work between replays
        torch.cuda.synchronize()


def _decode(layer, x, out, ids, wts):
    return layer.forward(x, out=out, ids=ids, wts=wts)


def _prefill(layer, x, out, ids, wts):
    return layer.prefill(x, out=out, ids=ids, wts=wts)


@pytest.mark.parametrize("et,st,M", [
    (O.Q4_0, O.Q4_0, 1),     # one-token kernels (config 3 types)
    (O.IQ3_S, O.Q8_0, 1),    # one-token kernels, IQ3_S experts
    (O.IQ3_S, O.Q8_0, 8),    # several-token kernels (config 4 types)
    (O.Q4_0, O.Q4_0, 5),
])
def test_decode_graph_replays(dev, et, st, M):
    print(f"graph decode et={et} st={st} M={M}", flush=True)
    layer = build(dev, 900 + M + et, et=et, st=st, gate_vec=True)
    _check_replays(layer, _decode, M, layer.H, layer.K, dev, 910 + M)


def test_decode_graph_kquant_shared(dev):
    """One token with the reference model's Q5_K shared expert."""
    import npref
    print("graph decode IQ3_S + Q5_K shared M=1", flush=True)
    E, K, H, F = 64, 8, 2048, 512
    g = torch.Generator(device=dev).manual_seed(920)
    router = torch.randn(E, H, generator=g, device=dev) * 0.02
    et = O.IQ3_S
    gate, up, down = qmat(et, F, H, E, g, dev), qmat(et, F, H, E, g, dev), qmat(et, H, F, E, g, dev)
    rng = np.random.default_rng(921)
    sh = tuple(torch.from_numpy(np.ascontiguousarray(npref.rand_kq(O.Q5_K, r, c, rng).reshape(-1))).to(dev)
               for r, c in ((F, H), (F, H), (H, F)))
    gw = torch.randn(H, generator=g, device=dev) * 0.02
    layer = MoeLayer(router, gate, up, down, et, K, shared=sh, shared_type=O.Q5_K, sh_gate_w=gw)
    _check_replays(layer, _decode, 1, H, K, dev, 922)


def test_prefill_graph_replays(dev):
    print("graph prefill Q4_0 T=96", flush=True)
    layer = build(dev, 930, E=64, et=O.Q4_0, st=O.Q4_0)
    T = 96
    layer.prefill(torch.zeros(T, layer.H, device=dev))   # sizes the workspace before capture
    _check_replays(layer, _prefill, T, layer.H, layer.K, dev, 931, order=1)


def test_gemv_sequence_graph_replays(dev):
    """The reference's per-layer GEMV sequence as ggml_gpu.rs issues it under
    capture: Q8_1 quantization, a Q4_0 GEMV, the fused f32 IQ3_S GEMV (own
    scratch), routing top-k and the batched IQ3_S expert GEMV on device ids."""
    from chimere_amd import ggml_gpu as G
    print("graph gemv sequence", flush=True)
    H, R, E, F, K = 2048, 1024, 32, 512, 8
    g = torch.Generator(device=dev).manual_seed(940)
    wq4 = qmat(O.Q4_0, R, H, 1, g, dev)[0]
    wiq = qmat(O.IQ3_S, R, H, 1, g, dev)[0]
    wexp = qmat(O.IQ3_S, F, H, E, g, dev)
    router = torch.randn(E, H, generator=g, device=dev) * 0.02
    x = torch.empty(H, device=dev)
    xq = torch.empty(G.q8_1_row_bytes(H), dtype=torch.uint8, device=dev)
    scratch = torch.empty_like(xq)
    y4, yi = torch.empty(R, device=dev), torch.empty(R, device=dev)
    logits = torch.empty(E, device=dev)
    ids = torch.empty(K, dtype=torch.int32, device=dev)
    wts = torch.empty(K, device=dev)
    ye = torch.empty(K, F, device=dev)

    def seq():
        G.ggml_gpu_quantize_q8_1(x, xq, H)
        G.ggml_gpu_gemv_q4_0_q8(wq4, xq, y4, R, H)
        G.ggml_gpu_gemv_iq3s_f32(wiq, x, yi, scratch, R, H)
        G.raw_f32_gemv(router, x, logits, E, H)
        G.gpu_topk_softmax(logits, ids, wts, E, K)
        G.ggml_gpu_gemv_iq3s_batched(wexp, xq, ye, ids, F, H, wexp.shape[1], 0, K)

    outs = (y4, yi, ids, wts, ye)
    inputs = [torch.randn(H, generator=g, device=dev) for _ in range(3)]
    want = []
    for xi in inputs:
        x.copy_(xi)
        seq()
        torch.cuda.synchronize()
        want.append([t.cpu().numpy().copy() for t in outs])
    x.copy_(inputs[0])
    gr = _capture(seq)
    for rep, i in enumerate([2, 0, 1, 2]):
        x.copy_(inputs[i])
        for t in (y4, yi, wts, ye):
            t.fill_(float("nan"))
        gr.replay()
        torch.cuda.synchronize()
        for j, t in enumerate(outs):
            assert np.array_equal(t.cpu().numpy(), want[i][j]), f"replay {rep} (input {i}): output {j} differs"
        x.copy_(torch.randn(H, generator=g, device=dev))   # eager work between replays
        seq()
        torch.cuda.synchronize()
