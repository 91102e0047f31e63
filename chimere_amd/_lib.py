"""ctypes binding of libchimere_hip.so (the C ABI declared in include/chimere_hip.h).

The library is built in-tree by ``make -C chimere_amd`` (``__graft_entry__.build()``).
Loading fails loudly when it is missing: there is no fallback implementation.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libchimere_hip.so")

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ3_S, MXFP4 = 2, 8, 12, 13, 14, 21, 39
TYPE_NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", IQ3_S: "iq3s", Q4_K: "q4k", Q5_K: "q5k", Q6_K: "q6k", MXFP4: "mxfp4"}

vp, i32, i64, f32p, szt = C.c_void_p, C.c_int, C.c_int64, C.c_void_p, C.c_size_t

# (name, restype, argtypes) for every symbol the header declares
SIGNATURES = [
    ("chimere_q8_1_block_bytes", i32, []),
    ("chimere_q8_1_block_elems", i32, []),
    ("chimere_matrix_row_padding", i32, []),
    ("chimere_quantize_q8_1", None, [vp, vp, i64, i64, vp]),
    ("chimere_quantize_q8_1_batched", None, [vp, vp, i64, i64, i32, vp]),
    ("chimere_mmvq_iq3s", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_q8_0", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_q4_0", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_q4_0_sform", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_iq3s_f32", None, [vp, vp, vp, i32, i32, i32, vp, vp]),
    ("chimere_mmvq_q8_0_f32", None, [vp, vp, vp, i32, i32, i32, vp, vp]),
    ("chimere_mmvq_q4_0_f32", None, [vp, vp, vp, i32, i32, i32, vp, vp]),
    ("chimere_mmvq_q5k", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_q4k", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_q6k", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_mxfp4", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_q5k_f32", None, [vp, vp, vp, i32, i32, i32, vp, vp]),
    ("chimere_mmvq_q4k_f32", None, [vp, vp, vp, i32, i32, i32, vp, vp]),
    ("chimere_mmvq_q6k_f32", None, [vp, vp, vp, i32, i32, i32, vp, vp]),
    ("chimere_mmvq_mxfp4_f32", None, [vp, vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_mmvq_mxfp4_batched", None, [vp, vp, vp, vp, i32, i32, i32, i64, i64, i32, vp]),
    ("chimere_mmvq_iq3s_batched", None, [vp, vp, vp, vp, i32, i32, i32, i64, i64, i32, vp]),
    ("chimere_mmvq_q8_0_batched", None, [vp, vp, vp, vp, i32, i32, i32, i64, i64, i32, vp]),
    ("chimere_mmvq_q4_0_batched", None, [vp, vp, vp, vp, i32, i32, i32, i64, i64, i32, vp]),
    ("chimere_mmvq_multi", None, [i32, vp, vp, vp, i32, i32, i32, i32, vp]),
    ("chimere_mmvq_q4_0_multi", None, [vp, vp, vp, i32, i32, i32, i32, vp]),
    ("chimere_mmvq_q8_0_multi", None, [vp, vp, vp, i32, i32, i32, i32, vp]),
    ("chimere_mmvq_iq3s_multi", None, [vp, vp, vp, i32, i32, i32, i32, vp]),
    ("chimere_f32_gemv", None, [vp, vp, vp, i32, i32, vp]),
    ("chimere_topk_softmax", None, [vp, vp, vp, i32, i32, i32, vp]),
    ("chimere_silu_mul_inplace", None, [vp, vp, i32, vp]),
    ("chimere_weighted_combine", None, [vp, vp, vp, i32, i32, vp]),
    ("chimere_sigmoid_gate_add", None, [vp, vp, vp, i32, vp]),
    ("chimere_moe_workspace_size", szt, [vp, i32]),
    ("chimere_moe_workspace_init", None, [vp, szt, vp]),
    ("chimere_moe_ffn_decode", None, [vp, vp, vp, i32, vp, vp, vp, szt, vp]),
    ("chimere_moe_ffn_decode_stage", None, [vp, vp, vp, i32, vp, szt, i32, vp]),
    ("chimere_moe_ffn_decode_noalloc", None, [vp, vp, vp, i32, vp, vp, vp]),
    ("chimere_moe_prefill_workspace_size", szt, [vp, i32]),
    ("chimere_moe_prefill", None, [vp, vp, vp, i32, vp, vp, vp, szt, vp]),
    ("chimere_fused_moe_iq3s_workspace_size", szt, [i32, i32, i32]),
    ("chimere_fused_moe_iq3s", None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i64, i64, i64, i32, vp, szt, vp]),
    ("chimere_quantize_weights", None, [i32, vp, vp, i64, vp]),
    ("chimere_dbg_block_dots", None, [i32, vp, vp, vp, i32, i32, vp]),
    ("chimere_hip_get_last_error", i32, []),
    ("chimere_hip_get_last_error_string", C.c_char_p, []),
]


class MoeLayerC(C.Structure):
    """Mirror of ``struct chimere_moe_layer``."""
    _fields_ = [("hidden", C.c_int), ("ffn", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
                ("expert_type", C.c_int), ("shared_type", C.c_int),
                ("router_w", vp), ("logit_bias", vp),
                ("gate_exps", vp), ("up_exps", vp), ("down_exps", vp),
                ("gate_stride", C.c_int64), ("up_stride", C.c_int64), ("down_stride", C.c_int64),
                ("sh_gate", vp), ("sh_up", vp), ("sh_down", vp), ("sh_gate_w", vp)]


_lib = None


class ChimereError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"chimere_hip error {code}: {msg}")
        self.code = code


def lib():
    """Load libchimere_hip.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `make -C chimere_amd` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check():
    """Raise ChimereError if the last C-ABI call on this thread recorded an error."""
    L = lib()
    msg = L.chimere_hip_get_last_error_string()
    code = L.chimere_hip_get_last_error()
    if code != 0:
        raise ChimereError(code, msg.decode() if msg else "")
