"""The ncmoe layer path (chimere-server/src/qwen35_model/moe_ffn.rs:1507-1591 and
the shared expert after it, :1597-1761) through MoeLayer.forward_ncmoe: router
and top-k on the device, the routed IQ3_S experts in libchimere_cpu.so, the
shared expert on the device.  Bar: routing indices and weights bit-exact and
the layer output bit-exact against oracle.moe_ncmoe, whose CPU part is pinned
in tests/test_ncmoe_cpu.py."""
import numpy as np
import pytest
import torch

import npref
import oracle as O
from chimere_amd import ggml_gpu as G
from chimere_amd.moe import MoeLayer
from routing_margin import assert_topk_margin

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def qmat(t, rows, cols, n, g, dev, scale=0.02):
    wf = torch.randn(n * rows, cols, generator=g, device=dev) * scale
    out = torch.empty(n * rows * O.row_bytes(t, cols), dtype=torch.uint8, device=dev)
    G.quantize_weights(t, wf, out)
    return out.view(n, -1)


@pytest.mark.parametrize("H,F,E,K,st,gate_vec,bias", [
    (2048, 512, 256, 8, O.Q5_K, True, False),     # the reference's layer: IQ3_S experts, Q5_K shared
    (1024, 512, 64, 8, O.Q8_0, False, True),
    (512, 256, 16, 4, None, False, False),
])
def test_forward_ncmoe_bit_exact(H, F, E, K, st, gate_vec, bias):
    dev = torch.device("cuda:0")
    print(f"ncmoe H={H} F={F} E={E} K={K} st={st}", flush=True)
    g = torch.Generator(device=dev).manual_seed(H + E)
    router = torch.randn(E, H, generator=g, device=dev) * 0.02
    gate, up, down = qmat(O.IQ3_S, F, H, E, g, dev), qmat(O.IQ3_S, F, H, E, g, dev), qmat(O.IQ3_S, H, F, E, g, dev)
    sh = None
    if st is not None:
        rng = np.random.default_rng(H)
        if st in (O.Q4_K, O.Q5_K, O.Q6_K):
            sh = tuple(torch.from_numpy(np.ascontiguousarray(npref.rand_kq(st, r, c, rng).reshape(-1))).to(dev)
                       for r, c in ((F, H), (F, H), (H, F)))
        else:
            sh = tuple(m[0] for m in (qmat(st, F, H, 1, g, dev), qmat(st, F, H, 1, g, dev), qmat(st, H, F, 1, g, dev)))
    gw = torch.randn(H, generator=g, device=dev) * 0.02 if gate_vec else None
    lb = torch.randn(E, generator=g, device=dev) * 0.5 if bias else None
    layer = MoeLayer(router, gate, up, down, O.IQ3_S, K, shared=sh, shared_type=st, sh_gate_w=gw, logit_bias=lb)
    layer.attach_cpu_experts(host(gate), host(up), host(down))
    shh = tuple(host(t) for t in sh) if sh is not None else None
    for rep in range(3):
        x = torch.randn(H, generator=g, device=dev)
        xh = host(x)
        lg = O.router(host(router), xh)
        if lb is not None:
            lg = lg + host(lb)
        assert_topk_margin(lg[None], K)
        out, ids, w = layer.forward_ncmoe(x, nthreads=4)
        oo, io, wo = O.moe_ncmoe(xh[None], host(router), host(gate), host(up), host(down), O.IQ3_S, K, sh=shh,
                                 sh_type=-1 if st is None else st, sh_gate_w=None if gw is None else host(gw),
                                 logit_bias=None if lb is None else host(lb), L=16, G=1)
        assert (host(ids) == io[0]).all(), "routing indices differ"
        assert (host(w).view(np.uint32) == wo[0].view(np.uint32)).all(), "routing weights differ"
        assert (host(out).view(np.uint32) == oo[0].view(np.uint32)).all(), f"output differs (rep {rep})"
        # the routed sum alone agrees with the GPU-resident layer to the
        # activation quantization (Q8_K here, Q8_1 there)
        full = layer.forward(x.reshape(1, H))
        n = np.linalg.norm(host(full))
        assert np.linalg.norm(host(out) - host(full)[0]) <= 0.03 * n
