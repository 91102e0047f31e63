"""GPU parity of the f32-activation IQ3_S expert FFN (chimere_fused_moe_iq3s,
the reference's fused_moe_iq3s: chimere-server/src/kernels/fused_moe.rs:261-468)
against the oracle in the kernels' fixed order, bit for bit, through the C ABI.

Covers the reference model's shape (H=2048, F=512, top-8), rows of one
superblock (110 bytes, 2-byte aligned: the unaligned staging), two staged
K chunks (H=4096), top-16, and the accumulate semantics (the output is added
to, as the reference's atomicAdd does); a graph replay with new inputs."""
import numpy as np
import pytest
import torch

import oracle as O
from chimere_amd import ggml_gpu as G
from chimere_amd.moe import fused_moe_iq3s

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stack(rows, cols, E, g, dev):
    wf = torch.randn(E * rows, cols, generator=g, device=dev) * 0.02
    out = torch.empty(E * rows * O.row_bytes(O.IQ3_S, cols), dtype=torch.uint8, device=dev)
    G.quantize_weights(O.IQ3_S, wf, out)
    return out.view(E, -1)


def case(dev, seed, H, F, E, K):
    g = torch.Generator(device=dev).manual_seed(seed)
    gate, up, down = stack(F, H, E, g, dev), stack(F, H, E, g, dev), stack(H, F, E, g, dev)
    x = torch.randn(H, generator=g, device=dev)
    ids = torch.randperm(E, generator=g, device=dev)[:K].to(torch.int32)
    wts = torch.rand(K, generator=g, device=dev) * 0.3 + 0.05
    out0 = torch.randn(H, generator=g, device=dev) * 0.1
    return gate, up, down, x, ids, wts, out0


def oracle_of(gate, up, down, x, ids, wts, out0, H, F):
    return O.fused_moe_iq3s(host(x), host(gate), host(up), host(down), host(ids), host(wts), host(out0).copy(),
                            H, F, gate.shape[1], up.shape[1], down.shape[1])


@pytest.mark.parametrize("H,F,E,K", [(2048, 512, 256, 8), (256, 256, 4, 1), (1024, 256, 16, 5), (4096, 512, 24, 16),
                                     (2048, 512, 64, 2)])
def test_fused_moe_iq3s_bit_exact(dev, H, F, E, K):
    print(f"fused_moe_iq3s H={H} F={F} E={E} K={K}", flush=True)
    gate, up, down, x, ids, wts, out0 = case(dev, H + F + E + K, H, F, E, K)
    out = out0.clone()
    fused_moe_iq3s(x, gate, up, down, ids, wts, out, H, F, gate.shape[1], up.shape[1], down.shape[1], K)
    want = oracle_of(gate, up, down, x, ids, wts, out0, H, F)
    got = host(out)
    assert (got.view(np.uint32) == want.view(np.uint32)).all(), np.abs(got - want).max()
    # accumulates: a second call adds the same FFN again (exactly, to the new output)
    fused_moe_iq3s(x, gate, up, down, ids, wts, out, H, F, gate.shape[1], up.shape[1], down.shape[1], K)
    want2 = O.fused_moe_iq3s(host(x), host(gate), host(up), host(down), host(ids), host(wts), want.copy(), H, F,
                             gate.shape[1], up.shape[1], down.shape[1])
    assert (host(out).view(np.uint32) == want2.view(np.uint32)).all()


def test_fused_moe_iq3s_graph_replays(dev):
    """Captured in a HIP graph, replayed with new activations / experts
    written into the captured buffers, eager work between replays; every
    replay bit-exact against the oracle."""
    H, F, E, K = 2048, 512, 32, 8
    gate, up, down, x, ids, wts, out0 = case(dev, 77, H, F, E, K)
    out = torch.zeros(H, device=dev)
    ws = torch.empty(K * F * 4, dtype=torch.uint8, device=dev)
    args = (H, F, gate.shape[1], up.shape[1], down.shape[1], K)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused_moe_iq3s(x, gate, up, down, ids, wts, out, *args, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        fused_moe_iq3s(x, gate, up, down, ids, wts, out, *args, workspace=ws)
    gen = torch.Generator(device=dev).manual_seed(5)
    for r in range(3):
        x.copy_(torch.randn(H, generator=gen, device=dev))
        ids.copy_(torch.randperm(E, generator=gen, device=dev)[:K].to(torch.int32))
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        got = host(out)
        want = oracle_of(gate, up, down, x, ids, wts, torch.zeros(H, device=dev), H, F)
        assert (got.view(np.uint32) == want.view(np.uint32)).all(), r
        torch.randn(1024, device=dev).sum()   # eager work between replays


def test_fused_moe_iq3s_repeated_ids(dev):
    """Expert ids are taken as given (the reference does no dedup either):
    a repeated expert contributes once per occurrence, in k order."""
    H, F, E, K = 1024, 512, 8, 5
    gate, up, down, x, _, wts, out0 = case(dev, 31, H, F, E, K)
    ids = torch.tensor([3, 3, 7, 3, 0], dtype=torch.int32, device=dev)
    out = out0.clone()
    fused_moe_iq3s(x, gate, up, down, ids, wts, out, H, F, gate.shape[1], up.shape[1], down.shape[1], K)
    want = oracle_of(gate, up, down, x, ids, wts, out0, H, F)
    assert (host(out).view(np.uint32) == want.view(np.uint32)).all()
