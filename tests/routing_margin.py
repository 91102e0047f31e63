"""Top-k ordering margin: when is a top-k selection independent of the
exponential used?

The reference selects experts by softmax probability computed with CUDA's
``expf`` (cs/kernels/chimere_kernels.cu:1185, 1203-1212); this library and
its oracle use their own deterministic exponential.  Both are applied to the
same reduced arguments d_i = fl(l_i - max) and then divided by each side's
own sum, and division by one positive value is monotone, so the two
selections (indices and their order) agree whenever consecutive entries of
the top K+1, sorted by logit, are separated in d by more than the two
exponentials' combined relative error can bridge:

    exp_a(d_i) / exp_b(d_{i+1}) > 1  whenever  d_i - d_{i+1} > r_a + r_b + 1 ulp

with r the relative error bound of each exponential: CUDA documents expf at
2 ulp (2.4e-7) and this library's measures 7.9e-8 (oracle exp scan).  The
margin required here, 1e-6, is about four times that sum.  Equal logits
(exact ties) are a separate contract: both sides pick the lowest index, and
then the reduced arguments are equal, so every exponential gives equal
probabilities.
"""
import numpy as np

EXP_ORDER_MARGIN = 1e-6


def reduced_args(logits):
    """fl32(l - max(l)) exactly as the kernels form it."""
    lg = np.asarray(logits, np.float32)
    return (lg - lg.max()).astype(np.float32)


def topk_margin(logits, K):
    """Smallest gap d_i - d_{i+1} among the K+1 largest reduced arguments
    (inf when K >= len(logits): every entry is selected)."""
    d = np.sort(reduced_args(logits).astype(np.float64))[::-1]
    if K >= d.size:
        return np.inf
    return float(np.min(d[:K] - d[1:K + 1]))


def assert_topk_margin(logits, K, what=""):
    for t, row in enumerate(np.atleast_2d(logits)):
        m = topk_margin(row, K)
        assert m > EXP_ORDER_MARGIN, (
            f"{what} token {t}: top-{K} gap {m:.3g} <= {EXP_ORDER_MARGIN}: selection could depend on the exp used")
