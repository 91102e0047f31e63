"""Host-side mirror of the reference's Rust wrapper module for this path,
``chimere-server/src/kernels/ggml_gpu.rs`` (extern decls :101-240, buffers
:292-406, wrappers :445-1488), over libchimere_hip.so.

Same function names, argument order and meaning (``nrows``/``ncols`` are the
GEMV's output/input sizes, strides are in bytes).  Arguments are torch tensors
on a ROCm device; every launch goes to the current torch stream (the
reference's ``global_stream()``).  Where the Rust wrapper returns
``Result<()>``, these raise ``ChimereError`` when the library rejected a call.
"""
import ctypes as C

import torch

from ._lib import IQ3_S, Q4_0, Q8_0, check, lib

Q8_1_BLOCK_BYTES = 36
Q8_1_BLOCK_ELEMS = 32
MATRIX_ROW_PADDING = 512


def pad(n, align):
    """ggml_gpu.rs:55"""
    return (n + align - 1) // align * align


def q8_1_row_bytes(ncols):
    return pad(ncols, MATRIX_ROW_PADDING) // Q8_1_BLOCK_ELEMS * Q8_1_BLOCK_BYTES


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


# ------------------------------------------------------------ quantize

def ggml_gpu_quantize_q8_1(input, q8_output, ncols):
    """ggml_gpu.rs:445 -- input f32[ncols] -> Q8_1 (padded to 512)."""
    lib().chimere_quantize_q8_1(_ptr(input), _ptr(q8_output), ncols, pad(ncols, MATRIX_ROW_PADDING), _stream())
    check()


def ggml_gpu_quantize_q8_1_batched(input, q8_output, ncols, batch):
    """ggml_gpu.rs:1282 -- batch contiguous rows of ncols."""
    lib().chimere_quantize_q8_1_batched(_ptr(input), _ptr(q8_output), ncols, pad(ncols, MATRIX_ROW_PADDING),
                                        batch, _stream())
    check()


# ---------------------------------------------------------------- GEMV

def _gemv_q8(name, weights, q8_input, output, nrows, ncols):
    nrows_y = pad(ncols, MATRIX_ROW_PADDING) // Q8_1_BLOCK_ELEMS
    getattr(lib(), name)(_ptr(weights), _ptr(q8_input), _ptr(output), ncols, nrows, nrows_y, _stream())
    check()


def ggml_gpu_gemv_iq3s_q8(weights, q8_input, output, nrows, ncols):
    """ggml_gpu.rs:714 -- pre-quantized Q8_1 input."""
    _gemv_q8("chimere_mmvq_iq3s", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_q8_0_q8(weights, q8_input, output, nrows, ncols):
    _gemv_q8("chimere_mmvq_q8_0", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_q4_0_q8(weights, q8_input, output, nrows, ncols):
    _gemv_q8("chimere_mmvq_q4_0", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_q4_0_sform_q8(weights, q8_input, output, nrows, ncols):
    """Q4_0 GEMV with ggml's s-form block term d_w*(sum(nib*q_x)*d_x - 8*s_x)
    (ggml-parity experiments; the default Q4_0 GEMV uses the exact integer form)."""
    _gemv_q8("chimere_mmvq_q4_0_sform", weights, q8_input, output, nrows, ncols)


def _gemv_f32(name, weights, input, output, q8_scratch, nrows, ncols):
    getattr(lib(), name)(_ptr(weights), _ptr(input), _ptr(output), ncols, nrows,
                         pad(ncols, MATRIX_ROW_PADDING), _ptr(q8_scratch), _stream())
    check()


def ggml_gpu_gemv_iq3s_f32(weights, input, output, q8_scratch, nrows, ncols):
    """ggml_gpu.rs:917 -- fused F32 -> Q8_1 -> IQ3_S GEMV."""
    _gemv_f32("chimere_mmvq_iq3s_f32", weights, input, output, q8_scratch, nrows, ncols)


def ggml_gpu_gemv_q8_0_f32(weights, input, output, q8_scratch, nrows, ncols):
    """ggml_gpu.rs:956"""
    _gemv_f32("chimere_mmvq_q8_0_f32", weights, input, output, q8_scratch, nrows, ncols)


def ggml_gpu_gemv_q4_0_f32(weights, input, output, q8_scratch, nrows, ncols):
    _gemv_f32("chimere_mmvq_q4_0_f32", weights, input, output, q8_scratch, nrows, ncols)


def ggml_gpu_gemv_q5k_q8(weights, q8_input, output, nrows, ncols):
    """ggml_gpu.rs:747 -- Q5_K weights, pre-quantized Q8_1 input."""
    _gemv_q8("chimere_mmvq_q5k", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_q4k_q8(weights, q8_input, output, nrows, ncols):
    _gemv_q8("chimere_mmvq_q4k", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_q6k_q8(weights, q8_input, output, nrows, ncols):
    _gemv_q8("chimere_mmvq_q6k", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_mxfp4_q8(weights, q8_input, output, nrows, ncols):
    _gemv_q8("chimere_mmvq_mxfp4", weights, q8_input, output, nrows, ncols)


def ggml_gpu_gemv_q5k_f32(weights, input, output, q8_scratch, nrows, ncols):
    """ggml_gpu.rs:834 -- fused F32 -> Q8_1 -> Q5_K GEMV."""
    _gemv_f32("chimere_mmvq_q5k_f32", weights, input, output, q8_scratch, nrows, ncols)


def ggml_gpu_gemv_q4k_f32(weights, input, output, q8_scratch, nrows, ncols):
    """ggml_gpu.rs:995"""
    _gemv_f32("chimere_mmvq_q4k_f32", weights, input, output, q8_scratch, nrows, ncols)


def ggml_gpu_gemv_q6k_f32(weights, input, output, q8_scratch, nrows, ncols):
    """ggml_gpu.rs:1034"""
    _gemv_f32("chimere_mmvq_q6k_f32", weights, input, output, q8_scratch, nrows, ncols)


def ggml_gpu_gemv_mxfp4_f32(weights, input, output, q8_scratch, nrows, ncols):
    """ggml_cuda_gemv.cu:448 (its argument order: scratch before output)."""
    lib().chimere_mmvq_mxfp4_f32(_ptr(weights), _ptr(input), _ptr(q8_scratch), _ptr(output), ncols, nrows,
                                 pad(ncols, MATRIX_ROW_PADDING), _stream())
    check()


def _gemv_batched(name, all_weights, q8_input, output, expert_ids, nrows, ncols, expert_stride,
                  input_stride, top_k):
    nrows_y = pad(ncols, MATRIX_ROW_PADDING) // Q8_1_BLOCK_ELEMS
    getattr(lib(), name)(_ptr(all_weights), _ptr(q8_input), _ptr(output), _ptr(expert_ids), ncols, nrows,
                         nrows_y, expert_stride, input_stride, top_k, _stream())
    check()


def ggml_gpu_gemv_iq3s_batched(all_weights, q8_input, output, expert_ids, nrows, ncols, expert_stride,
                               input_stride, top_k):
    """ggml_gpu.rs:1225 -- top_k expert GEMVs with device-resident ids."""
    _gemv_batched("chimere_mmvq_iq3s_batched", all_weights, q8_input, output, expert_ids, nrows, ncols,
                  expert_stride, input_stride, top_k)


def ggml_gpu_gemv_q8_0_batched(all_weights, q8_input, output, expert_ids, nrows, ncols, expert_stride,
                               input_stride, top_k):
    _gemv_batched("chimere_mmvq_q8_0_batched", all_weights, q8_input, output, expert_ids, nrows, ncols,
                  expert_stride, input_stride, top_k)


def ggml_gpu_gemv_q4_0_batched(all_weights, q8_input, output, expert_ids, nrows, ncols, expert_stride,
                               input_stride, top_k):
    _gemv_batched("chimere_mmvq_q4_0_batched", all_weights, q8_input, output, expert_ids, nrows, ncols,
                  expert_stride, input_stride, top_k)


def ggml_gpu_gemv_mxfp4_batched(all_weights, q8_input, output, expert_ids, nrows, ncols, expert_stride,
                                input_stride, top_k):
    """ggml_cuda_gemv.cu:425 with device-resident ids."""
    _gemv_batched("chimere_mmvq_mxfp4_batched", all_weights, q8_input, output, expert_ids, nrows, ncols,
                  expert_stride, input_stride, top_k)


def gemv_multi(wtype, weights, q8_input, output, nrows, ncols, ntok):
    """M <= 8 tokens against one dense matrix; q8_input rows of q8_1_row_bytes(ncols)."""
    nrows_y = pad(ncols, MATRIX_ROW_PADDING) // Q8_1_BLOCK_ELEMS
    lib().chimere_mmvq_multi(wtype, _ptr(weights), _ptr(q8_input), _ptr(output), ncols, nrows, nrows_y, ntok,
                             _stream())
    check()


def block_dots(wtype, weights, q8_input, out_i32, nrows, ncols):
    """Exact int32 per-block dots (debug entry point)."""
    lib().chimere_dbg_block_dots(wtype, _ptr(weights), _ptr(q8_input), _ptr(out_i32), ncols, nrows, _stream())
    check()


def quantize_weights(wtype, x_f32, out_u8):
    lib().chimere_quantize_weights(wtype, _ptr(x_f32), _ptr(out_u8), x_f32.numel(), _stream())
    check()


# ------------------------------------------------------ routing / glue

def raw_f32_gemv(A, x, y, rows, cols):
    """elementwise.rs:599 raw_f32_gemv"""
    lib().chimere_f32_gemv(_ptr(A), _ptr(x), _ptr(y), rows, cols, _stream())
    check()


def gpu_topk_softmax(logits, top_indices, top_weights, num_experts, top_k, ntok=1):
    """topk_softmax.rs:113"""
    lib().chimere_topk_softmax(_ptr(logits), _ptr(top_indices), _ptr(top_weights), num_experts, top_k, ntok,
                               _stream())
    check()


def silu_mul_inplace(gate, up, n):
    """fused_ops.rs:34 / silu_mul_inplace_slices"""
    lib().chimere_silu_mul_inplace(_ptr(gate), _ptr(up), n, _stream())
    check()


def weighted_combine_gpu(expert_outputs, weights, accum, hidden_size, top_k):
    """fused_ops.rs:364"""
    lib().chimere_weighted_combine(_ptr(expert_outputs), _ptr(weights), _ptr(accum), hidden_size, top_k,
                                   _stream())
    check()


def raw_sigmoid_gate_add_inplace(output, gate, combined, n):
    """scratch_pool.rs:264"""
    lib().chimere_sigmoid_gate_add(_ptr(output), _ptr(gate), _ptr(combined), n, _stream())
    check()


class GgmlGpuBuffers:
    """ggml_gpu.rs:292-406 -- preallocated Q8_1 / batched MoE scratch."""

    def __init__(self, max_ncols, max_nrows, expert_ffn=0, hidden_size=0, top_k=0, device="cuda"):
        self.max_ncols_padded = pad(max_ncols, MATRIX_ROW_PADDING)
        u8 = dict(dtype=torch.uint8, device=device)
        f32 = dict(dtype=torch.float32, device=device)
        self.q8_input = torch.zeros(self.max_ncols_padded // 32 * 36, **u8)
        self.q8_input_b = torch.zeros(self.max_ncols_padded // 32 * 36, **u8)
        self.output = torch.zeros(max_nrows, **f32)
        self.batched_gate = torch.zeros(max(top_k * expert_ffn, 1), **f32)
        self.batched_up = torch.zeros(max(top_k * expert_ffn, 1), **f32)
        self.batched_down = torch.zeros(max(top_k * hidden_size, 1), **f32)
        self.batched_q8_inter = torch.zeros(max(top_k * q8_1_row_bytes(max(expert_ffn, 1)), 1), **u8)

    @classmethod
    def with_moe(cls, max_ncols, max_nrows, expert_ffn, hidden_size, top_k, device="cuda"):
        return cls(max_ncols, max_nrows, expert_ffn, hidden_size, top_k, device)


__all__ = [n for n in dir() if not n.startswith("_")] + ["IQ3_S", "Q4_0", "Q8_0"]
