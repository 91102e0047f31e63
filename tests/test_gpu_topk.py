"""GPU parity of the standalone softmax + top-k (chimere_topk_softmax,
topk_softmax.rs:113 / cs/kernels/chimere_kernels.cu:1150-1223) against the
CPU oracle, through the C ABI: indices and weights bit-exact, including
exact probability ties that straddle the top-k boundary (lowest index
first, as the reference's strict '>' arg-max rounds give)."""
import numpy as np
import pytest
import torch

import oracle as O
from chimere_amd import ggml_gpu as G

pytestmark = pytest.mark.gpu


def _cases(E, seed):
    rng = np.random.default_rng(seed)
    yield rng.standard_normal(E).astype(np.float32)                     # distinct
    yield np.zeros(E, np.float32)                                       # all tied
    v = rng.standard_normal(E // 2).astype(np.float32)
    yield np.repeat(v, 2)                                               # pairs tied
    yield np.round(rng.standard_normal(E) * 2).astype(np.float32)       # few distinct values
    v = np.full(E, -1.0, np.float32)
    v[rng.choice(E, 3, replace=False)] = 2.0                            # 3 winners, then a tie of E-3
    yield v
    v = rng.standard_normal(E).astype(np.float32)
    v[::7] = v.max()                                                    # many copies of the maximum
    yield v
    yield (rng.standard_normal(E) * 40).astype(np.float32)              # probabilities underflow to 0


@pytest.mark.parametrize("E,K", [(256, 8), (256, 1), (256, 4), (256, 16), (200, 8), (130, 16), (64, 8), (8, 8),
                                 (512, 16), (1024, 8)])
def test_topk_softmax_ties(E, K):
    print(f"topk E={E} K={K}", flush=True)
    rows = list(_cases(E, E * 100 + K))
    logits = np.stack(rows)
    n = len(rows)
    dl = torch.from_numpy(logits).cuda()
    ids = torch.empty(n, K, dtype=torch.int32, device="cuda")
    wts = torch.empty(n, K, dtype=torch.float32, device="cuda")
    G.gpu_topk_softmax(dl, ids, wts, E, K, ntok=n)
    torch.cuda.synchronize()
    gi, gw = ids.cpu().numpy(), wts.cpu().numpy()
    for t in range(n):
        oi, ow = O.topk_softmax(logits[t], K)
        assert (gi[t] == oi).all(), (t, gi[t], oi)
        assert (gw[t].view(np.uint32) == ow.view(np.uint32)).all(), (t, gw[t], ow)


def test_device_exp_equals_oracle_over_softmax_range():
    """K = E = 16: every probability is returned, so the device exponential
    is compared with the oracle's on 61440 arguments spread over [-87, 0]
    (the softmax range; one logit per row is the maximum, 0)."""
    E = K = 16
    rng = np.random.default_rng(16)
    n = 4096
    logits = rng.uniform(-87.0, 0.0, (n, E)).astype(np.float32)
    logits[:, 0] = 0.0
    logits[: n // 2, 1:] = rng.uniform(-1.0, 0.0, (n // 2, E - 1)).astype(np.float32)   # dense near 0
    dl = torch.from_numpy(logits).cuda()
    ids = torch.empty(n, K, dtype=torch.int32, device="cuda")
    wts = torch.empty(n, K, dtype=torch.float32, device="cuda")
    G.gpu_topk_softmax(dl, ids, wts, E, K, ntok=n)
    torch.cuda.synchronize()
    gi, gw = ids.cpu().numpy(), wts.cpu().numpy()
    for t in range(n):
        oi, ow = O.topk_softmax(logits[t], K)
        assert (gi[t] == oi).all() and (gw[t].view(np.uint32) == ow.view(np.uint32)).all(), t


@pytest.mark.parametrize("E,K", [(256, 8), (256, 16), (256, 2), (160, 8)])
def test_topk_softmax_many_tied_rows(E, K):
    """2048 rows of logits on a coarse grid (many exact ties at every rank,
    including the K-th) and 2048 of continuous logits, against the oracle."""
    print(f"topk many rows E={E} K={K}", flush=True)
    rng = np.random.default_rng(E * 7 + K)
    n = 4096
    logits = np.empty((n, E), np.float32)
    logits[: n // 2] = rng.integers(-3, 4, (n // 2, E)).astype(np.float32) * 0.5
    logits[n // 2:] = rng.standard_normal((n - n // 2, E)).astype(np.float32)
    dl = torch.from_numpy(logits).cuda()
    ids = torch.empty(n, K, dtype=torch.int32, device="cuda")
    wts = torch.empty(n, K, dtype=torch.float32, device="cuda")
    G.gpu_topk_softmax(dl, ids, wts, E, K, ntok=n)
    torch.cuda.synchronize()
    gi, gw = ids.cpu().numpy(), wts.cpu().numpy()
    for t in range(n):
        oi, ow = O.topk_softmax(logits[t], K)
        assert (gi[t] == oi).all(), (t, gi[t], oi)
        assert (gw[t].view(np.uint32) == ow.view(np.uint32)).all(), (t, gw[t], ow)
