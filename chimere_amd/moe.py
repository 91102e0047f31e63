"""MoE FFN layer over libchimere_hip.so.

``MoeLayer`` holds one layer's device weights (stacked expert tensors in the
reference's GGUF block layout) and a preallocated workspace, and runs
``chimere_moe_ffn_decode`` (router -> top-k -> gate/up+SiLU -> down ->
weighted sum + shared expert) for 1..8 tokens, or ``chimere_moe_prefill``
for a chunk of tokens.

``forward_ncmoe`` runs one token with the routed experts on the host
(``chimere_amd.cpu``, the reference's "ncmoe" path) and the rest on the
device.

``fused_moe_iq3s`` is the expert FFN on unquantized activations (the
reference's fallback GPU path, ``chimere-server/src/kernels/fused_moe.rs``).

``forward_moe_v3`` replays the reference's own launch sequence
(``chimere-server/src/qwen35_model/moe_ffn.rs:1094-1384`` V3 batched path and
``:1597-1761`` shared expert) through the ``ggml_gpu`` mirror; it computes the
same values as the fused entry point and serves as its cross-check.
"""
import ctypes as C

import torch

from . import ggml_gpu as G
from ._lib import IQ3_S, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, MoeLayerC, check, lib

_BLOCK = {Q8_0: (32, 34), Q4_0: (32, 18), IQ3_S: (256, 110)}


def row_bytes(wtype, ncols):
    e, b = _BLOCK[wtype]
    return ncols // e * b


class MoeLayer:
    """One routed-MoE layer.

    router_w [E, H] f32; gate/up [E, F*row_bytes(H)] u8; down [E, H*row_bytes(F)] u8;
    shared = (gate [F*rb(H)], up, down [H*rb(F)]) u8 or None; sh_gate_w [H] f32 or None;
    logit_bias [E] f32 or None.  All tensors on the same ROCm device.
    """

    def __init__(self, router_w, gate, up, down, expert_type, top_k, shared=None, shared_type=None,
                 sh_gate_w=None, logit_bias=None, max_ntok=8):
        E, H = router_w.shape
        self.H, self.E, self.K = H, E, top_k
        self.expert_type = expert_type
        self.F = gate.numel() // E // row_bytes(expert_type, H)
        self.shared_type = shared_type if shared is not None else -1
        self.tensors = [router_w, gate, up, down, sh_gate_w, logit_bias] + list(shared or [])
        self.c = MoeLayerC()
        c = self.c
        c.hidden, c.ffn, c.n_experts, c.top_k = H, self.F, E, top_k
        c.expert_type, c.shared_type = expert_type, self.shared_type
        c.router_w = router_w.data_ptr()
        c.logit_bias = logit_bias.data_ptr() if logit_bias is not None else None
        c.gate_exps, c.up_exps, c.down_exps = gate.data_ptr(), up.data_ptr(), down.data_ptr()
        c.gate_stride = gate.numel() // E
        c.up_stride = up.numel() // E
        c.down_stride = down.numel() // E
        if shared is not None:
            c.sh_gate, c.sh_up, c.sh_down = (t.data_ptr() for t in shared)
        c.sh_gate_w = sh_gate_w.data_ptr() if sh_gate_w is not None else None
        self.max_ntok = max_ntok
        self.ws_bytes = lib().chimere_moe_workspace_size(C.byref(c), max_ntok)
        if self.ws_bytes == 0:
            raise ValueError("chimere_moe_workspace_size rejected the layer shape")
        self.workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=router_w.device)
        lib().chimere_moe_workspace_init(C.c_void_p(self.workspace.data_ptr()), self.ws_bytes, G._stream())
        check()
        self.device = router_w.device

    def forward(self, x, out=None, ids=None, wts=None):
        """x [M, H] f32 (M <= max_ntok) -> out [M, H]; ids/wts [M, K] optional outputs."""
        M = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        lib().chimere_moe_ffn_decode(C.byref(self.c), C.c_void_p(x.data_ptr()), C.c_void_p(out.data_ptr()), M,
                                     C.c_void_p(ids.data_ptr()) if ids is not None else None,
                                     C.c_void_p(wts.data_ptr()) if wts is not None else None,
                                     C.c_void_p(self.workspace.data_ptr()), self.ws_bytes, G._stream())
        check()
        return out

    def forward_noalloc(self, x, out=None, ids=None, wts=None):
        """forward() through chimere_moe_ffn_decode_noalloc (the library's static
        per-device scratch instead of this layer's workspace)."""
        if out is None:
            out = torch.empty_like(x)
        lib().chimere_moe_ffn_decode_noalloc(C.byref(self.c), C.c_void_p(x.data_ptr()), C.c_void_p(out.data_ptr()),
                                             x.shape[0], C.c_void_p(ids.data_ptr()) if ids is not None else None,
                                             C.c_void_p(wts.data_ptr()) if wts is not None else None, G._stream())
        check()
        return out

    def prefill(self, x, out=None, ids=None, wts=None):
        """x [T, H] f32, any T >= 1 -> out [T, H] through chimere_moe_prefill
        (int8 matrix-core grouped GEMMs; Q4_0 / Q8_0 / IQ3_S experts, the shared expert
        also Q4_K / Q5_K / Q6_K).  The prefill
        workspace is allocated on first use and grown when T exceeds it."""
        T = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        if getattr(self, "pf_ntok", 0) < T:
            self.pf_bytes = lib().chimere_moe_prefill_workspace_size(C.byref(self.c), T)
            if self.pf_bytes == 0:
                raise ValueError("chimere_moe_prefill_workspace_size rejected the layer shape")
            self.pf_workspace = torch.empty(self.pf_bytes, dtype=torch.uint8, device=self.device)
            self.pf_ntok = T
        lib().chimere_moe_prefill(C.byref(self.c), C.c_void_p(x.data_ptr()), C.c_void_p(out.data_ptr()), T,
                                  C.c_void_p(ids.data_ptr()) if ids is not None else None,
                                  C.c_void_p(wts.data_ptr()) if wts is not None else None,
                                  C.c_void_p(self.pf_workspace.data_ptr()), self.pf_bytes, G._stream())
        check()
        return out

    # ------------------------------------------------------------------
    def _route(self, x, bufs):
        """Router GEMV (+ bias) and top-k softmax on the device (moe_ffn.rs:1094-1140)."""
        E, K, dev = self.E, self.K, self.device
        router_w, logit_bias = self.tensors[0], self.tensors[5]
        router_out = torch.empty(E, dtype=torch.float32, device=dev)
        ids = torch.empty(K, dtype=torch.int32, device=dev)
        w = torch.empty(K, dtype=torch.float32, device=dev)
        G.raw_f32_gemv(router_w, x, router_out, E, self.H)
        if logit_bias is not None:
            router_out += logit_bias
        G.gpu_topk_softmax(router_out, ids, w, E, K)
        return ids, w

    def _shared_tail(self, x, accum, bufs):
        """Shared expert on the device, combined with the routed sum `accum`
        (moe_ffn.rs:1597-1761); returns `accum` alone without a shared expert."""
        if self.shared_type < 0:
            return accum
        H, F, dev = self.H, self.F, self.device
        sh_gate_w = self.tensors[4]
        sg, su, sd = self.tensors[6:9]
        st = self.shared_type
        f32 = {Q8_0: G.ggml_gpu_gemv_q8_0_f32, Q4_0: G.ggml_gpu_gemv_q4_0_f32, IQ3_S: G.ggml_gpu_gemv_iq3s_f32,
               Q4_K: G.ggml_gpu_gemv_q4k_f32, Q5_K: G.ggml_gpu_gemv_q5k_f32, Q6_K: G.ggml_gpu_gemv_q6k_f32}[st]
        q8 = {Q8_0: G.ggml_gpu_gemv_q8_0_q8, Q4_0: G.ggml_gpu_gemv_q4_0_q8, IQ3_S: G.ggml_gpu_gemv_iq3s_q8,
              Q4_K: G.ggml_gpu_gemv_q4k_q8, Q5_K: G.ggml_gpu_gemv_q5k_q8, Q6_K: G.ggml_gpu_gemv_q6k_q8}[st]
        shg = torch.empty(F, dtype=torch.float32, device=dev)
        shu = torch.empty(F, dtype=torch.float32, device=dev)
        shd = torch.empty(H, dtype=torch.float32, device=dev)
        f32(sg, x, shg, bufs.q8_input, F, H)
        q8(su, bufs.q8_input, shu, F, H)
        G.silu_mul_inplace(shg, shu, F)
        f32(sd, shg, shd, bufs.q8_input_b, H, F)
        if sh_gate_w is not None:
            glogit = torch.empty(1, dtype=torch.float32, device=dev)
            G.raw_f32_gemv(sh_gate_w, x, glogit, 1, H)
            G.raw_sigmoid_gate_add_inplace(shd, glogit, accum, H)
        else:
            shd += accum
        return shd

    def forward_moe_v3(self, x):
        """One token through the reference's 7-launch V3 sequence + shared expert."""
        assert x.numel() == self.H
        H, F, E, K, t = self.H, self.F, self.E, self.K, self.expert_type
        dev = self.device
        gate, up, down = self.tensors[1:4]
        bufs = G.GgmlGpuBuffers.with_moe(max(H, F), max(H, F), F, H, K, device=dev)
        ids, w = self._route(x, bufs)
        G.ggml_gpu_quantize_q8_1(x, bufs.q8_input, H)
        bat = {Q8_0: G.ggml_gpu_gemv_q8_0_batched, Q4_0: G.ggml_gpu_gemv_q4_0_batched,
               IQ3_S: G.ggml_gpu_gemv_iq3s_batched}[t]
        bat(gate, bufs.q8_input, bufs.batched_gate, ids, F, H, gate.numel() // E, 0, K)
        bat(up, bufs.q8_input, bufs.batched_up, ids, F, H, up.numel() // E, 0, K)
        G.silu_mul_inplace(bufs.batched_gate, bufs.batched_up, K * F)
        G.ggml_gpu_quantize_q8_1_batched(bufs.batched_gate, bufs.batched_q8_inter, F, K)
        bat(down, bufs.batched_q8_inter, bufs.batched_down, ids, H, F, down.numel() // E,
            G.q8_1_row_bytes(F), K)
        accum = torch.empty(H, dtype=torch.float32, device=dev)
        G.weighted_combine_gpu(bufs.batched_down, w, accum, H, K)
        return self._shared_tail(x, accum, bufs), ids, w

    # ------------------------------------------------------------------
    def attach_cpu_experts(self, gate, up, down):
        """Host copies of the routed expert tensors for forward_ncmoe (the
        reference's gate_exps_cpu / up_exps_cpu / down_exps_cpu): numpy uint8
        [E, expert_bytes] in the device tensors' layout; IQ3_S only."""
        import numpy as np
        if self.expert_type != IQ3_S:
            raise ValueError("the CPU expert path takes IQ3_S experts only")
        arrs = tuple(np.ascontiguousarray(a, np.uint8).reshape(self.E, -1) for a in (gate, up, down))
        for a, t in zip(arrs, self.tensors[1:4]):
            if a.size != t.numel():
                raise ValueError("host expert tensor size differs from the device tensor")
        self.cpu_experts = arrs
        pin = torch.cuda.is_available()
        self._h_x = torch.empty(self.H, dtype=torch.float32, pin_memory=pin)
        self._h_ids = torch.empty(self.K, dtype=torch.int32, pin_memory=pin)
        self._h_w = torch.empty(self.K, dtype=torch.float32, pin_memory=pin)
        self._h_acc = torch.empty(self.H, dtype=torch.float32, pin_memory=pin)

    def _nc_capture(self):
        """HIP graphs of the device parts of forward_ncmoe: routing (from the
        static input buffer to ids / weights) and the shared-expert tail (from
        the static input and routed-sum buffers to the output)."""
        H, F, K, dev = self.H, self.F, self.K, self.device
        bufs = self._nc_bufs = G.GgmlGpuBuffers.with_moe(max(H, F), max(H, F), F, H, K, device=dev)
        self._nc_x = torch.zeros(H, dtype=torch.float32, device=dev)
        self._nc_accum = torch.zeros(H, dtype=torch.float32, device=dev)
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):                      # first calls outside capture
            self._route(self._nc_x, bufs)
            self._shared_tail(self._nc_x, self._nc_accum, bufs)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize(dev)
        self._g_route = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._g_route):
            self._nc_ids, self._nc_w = self._route(self._nc_x, bufs)
        self._g_tail = None                             # no shared expert: the routed sum is the output
        self._nc_out = self._nc_accum
        if self.shared_type >= 0:
            self._g_tail = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self._g_tail):
                self._nc_out = self._shared_tail(self._nc_x, self._nc_accum, bufs)

    def forward_ncmoe(self, x, nthreads=4):
        """One token with the routed experts on the host (moe_ffn.rs:1507-1591):
        router and top-k on the device, then hidden state, ids and weights to
        the host, libchimere_cpu.so's expert loop, the sum back to the device
        and the shared expert there.  The device parts replay two captured
        HIP graphs.  Returns (out [H], ids [K], weights [K]): buffers of this
        layer that the next call overwrites."""
        from . import cpu
        if not hasattr(self, "cpu_experts"):
            raise RuntimeError("attach_cpu_experts() first")
        assert x.numel() == self.H
        H, F = self.H, self.F
        if not hasattr(self, "_g_route"):
            self._nc_capture()
        self._nc_x.copy_(x.reshape(H))
        self._g_route.replay()
        self._h_ids.copy_(self._nc_ids, non_blocking=True)
        self._h_w.copy_(self._nc_w, non_blocking=True)
        self._h_x.copy_(self._nc_x, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()     # the host reads these next
        g, u, d = self.cpu_experts
        cpu.ncmoe_experts(g, u, d, self._h_ids.numpy(), self._h_w.numpy(), self._h_x.numpy(), H, F,
                          out=self._h_acc.numpy(), nthreads=nthreads)
        # stream-ordered: the next call's synchronize also covers this copy
        # before _h_acc is written again
        self._nc_accum.copy_(self._h_acc, non_blocking=True)
        if self._g_tail is not None:
            self._g_tail.replay()
        return self._nc_out, self._nc_ids, self._nc_w


def fused_moe_iq3s(hidden, gate_exps, up_exps, down_exps, expert_ids, expert_weights, output, hidden_size,
                   expert_ffn, expert_bytes_gate, expert_bytes_up, expert_bytes_down, top_k, workspace=None):
    """output [hidden_size] f32 += sum_k expert_weights[k] * FFN_{expert_ids[k]}(hidden): IQ3_S experts on
    the f32 hidden state through ``chimere_fused_moe_iq3s`` (the arguments of the reference's
    ``fused_moe_iq3s_gpu_resident``, chimere-server/src/kernels/fused_moe.rs:417-468; ids and weights are
    device tensors).  As there, output accumulates: zero it for the bare FFN.  The workspace (h of
    every expert) is allocated here unless one is passed."""
    need = lib().chimere_fused_moe_iq3s_workspace_size(hidden_size, expert_ffn, top_k)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=output.device)
    lib().chimere_fused_moe_iq3s(C.c_void_p(hidden.data_ptr()), C.c_void_p(gate_exps.data_ptr()),
                                 C.c_void_p(up_exps.data_ptr()), C.c_void_p(down_exps.data_ptr()),
                                 C.c_void_p(expert_ids.data_ptr()), C.c_void_p(expert_weights.data_ptr()),
                                 C.c_void_p(output.data_ptr()), hidden_size, expert_ffn, expert_bytes_gate,
                                 expert_bytes_up, expert_bytes_down, top_k, C.c_void_p(workspace.data_ptr()),
                                 workspace.numel(), G._stream())
    check()
    return output
