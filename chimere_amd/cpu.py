"""Host-side expert path ("ncmoe") over libchimere_cpu.so (include/chimere_cpu.h).

Mirrors the reference's safe Rust wrappers of its ggml IQ3_S wrapper
(chimere-server/ffi/src/lib.rs:690-845: ``iq3s_row_bytes``,
``iq3s_gemv_cpu``, ``iq3s_gemv_cpu_parallel``, ``iq3s_swiglu_expert_cpu``) with
the same names, argument order and panics (here: exceptions), plus
``ncmoe_experts`` -- the per-token expert loop of
chimere-server/src/qwen35_model/moe_ffn.rs:1507-1591 as one native call.

All arrays are host numpy arrays.  The library is built in-tree by
``make -C chimere_amd``; loading fails loudly when it is missing.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libchimere_cpu.so")
IQ3S_BLOCK_ELEMS, IQ3S_BLOCK_BYTES, Q8K_BLOCK_BYTES = 256, 110, 296

vp, i32, i64, szt = C.c_void_p, C.c_int, C.c_int64, C.c_size_t

SIGNATURES = [
    ("ggml_ffi_quantize_q8_K", None, [vp, vp, i64]),
    ("ggml_ffi_vec_dot_iq3s_q8K", None, [i32, vp, vp, vp]),
    ("ggml_ffi_gemv_iq3s", None, [vp, vp, vp, i32, i32]),
    ("ggml_ffi_gemv_iq3s_parallel", None, [vp, vp, vp, i32, i32, i32]),
    ("ggml_ffi_iq3s_row_bytes", szt, [i32]),
    ("ggml_ffi_q8k_row_bytes", szt, [i32]),
    ("chimere_ncmoe_experts", i32, [vp, vp, vp, szt, szt, szt, vp, vp, i32, vp, vp, i32, i32, i32, i32]),
    ("chimere_cpu_isa", i32, []),
]

_lib = None


def lib():
    """Load libchimere_cpu.so (raises if it was not built)."""
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


def _p(a):
    return C.c_void_p(a.ctypes.data)


def iq3s_row_bytes(ncols):
    return int(lib().ggml_ffi_iq3s_row_bytes(int(ncols)))


def quantize_q8_K(x):
    """f32 [k] (k % 256 == 0) -> Q8_K bytes [k / 256 * 296]."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    if x.size % IQ3S_BLOCK_ELEMS:
        raise ValueError("length must be a multiple of 256")
    y = np.empty(x.size // IQ3S_BLOCK_ELEMS * Q8K_BLOCK_BYTES, np.uint8)
    lib().ggml_ffi_quantize_q8_K(_p(x), _p(y), x.size)
    return y


def vec_dot_iq3s_q8K(n, vx, vy):
    s = C.c_float()
    vx, vy = np.ascontiguousarray(vx, np.uint8), np.ascontiguousarray(vy, np.uint8)
    if vx.size < n // 256 * IQ3S_BLOCK_BYTES or vy.size < n // 256 * Q8K_BLOCK_BYTES:
        raise ValueError("blocks too short")
    lib().ggml_ffi_vec_dot_iq3s_q8K(int(n), C.byref(s), _p(vx), _p(vy))
    return s.value


def _check_gemv(weights_iq3s, input_f32, nrows, ncols):
    if ncols % IQ3S_BLOCK_ELEMS:
        raise ValueError(f"ncols must be multiple of {IQ3S_BLOCK_ELEMS}")
    if input_f32.size < ncols:
        raise ValueError(f"input too short: {input_f32.size} < {ncols}")
    need = nrows * iq3s_row_bytes(ncols)
    if weights_iq3s.size < need:
        raise ValueError(f"weights too short: {weights_iq3s.size} < {need} ({nrows} rows x {ncols} cols)")


def iq3s_gemv_cpu(weights_iq3s, input_f32, nrows, ncols):
    """y[nrows] = W x, one thread (ffi/src/lib.rs:710-737)."""
    w = np.ascontiguousarray(weights_iq3s, np.uint8).ravel()
    x = np.ascontiguousarray(input_f32, np.float32).ravel()
    _check_gemv(w, x, nrows, ncols)
    y = np.zeros(nrows, np.float32)
    lib().ggml_ffi_gemv_iq3s(_p(w), _p(x), _p(y), nrows, ncols)
    return y


def iq3s_gemv_cpu_parallel(weights_iq3s, input_f32, nrows, ncols, nthreads):
    """y[nrows] = W x over nthreads OpenMP threads (ffi/src/lib.rs:747-777)."""
    w = np.ascontiguousarray(weights_iq3s, np.uint8).ravel()
    x = np.ascontiguousarray(input_f32, np.float32).ravel()
    _check_gemv(w, x, nrows, ncols)
    y = np.zeros(nrows, np.float32)
    lib().ggml_ffi_gemv_iq3s_parallel(_p(w), _p(x), _p(y), nrows, ncols, int(nthreads))
    return y


def iq3s_swiglu_expert_cpu(gate_w, up_w, down_w, input_f32, expert_ffn, hidden_size):
    """down(silu(gate x) * up x) for one expert (ffi/src/lib.rs:803-845):
    the expert loop with one expert of weight 1."""
    out = np.zeros(hidden_size, np.float32)
    ncmoe_experts(np.ascontiguousarray(gate_w, np.uint8).ravel()[None],
                  np.ascontiguousarray(up_w, np.uint8).ravel()[None],
                  np.ascontiguousarray(down_w, np.uint8).ravel()[None],
                  np.zeros(1, np.int32), np.ones(1, np.float32), input_f32, hidden_size, expert_ffn, out=out,
                  nthreads=1)
    return out


def ncmoe_experts(gate_exps, up_exps, down_exps, ids, weights, hidden, hidden_size, expert_ffn, out=None,
                  nthreads=4):
    """combined[H] = sum_k weights[k] * down_e(silu(gate_e h) * up_e h), e = ids[k]
    (moe_ffn.rs:1538-1585; the reference runs each GEMV on 4 threads).
    gate_exps/up_exps/down_exps: host uint8 [E, expert_bytes]."""
    gate_exps, up_exps, down_exps = (np.ascontiguousarray(a, np.uint8) for a in (gate_exps, up_exps, down_exps))
    E = gate_exps.shape[0]
    if up_exps.shape[0] != E or down_exps.shape[0] != E:
        raise ValueError("expert tensors disagree on the expert count")
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    weights = np.ascontiguousarray(weights, np.float32).ravel()
    hidden = np.ascontiguousarray(hidden, np.float32).ravel()
    if weights.size != ids.size or hidden.size < hidden_size:
        raise ValueError("ids/weights/hidden sizes")
    if out is None:
        out = np.empty(hidden_size, np.float32)
    rc = lib().chimere_ncmoe_experts(_p(gate_exps), _p(up_exps), _p(down_exps), gate_exps[0].size,
                                     up_exps[0].size, down_exps[0].size, _p(ids), _p(weights), ids.size,
                                     _p(hidden), _p(out), hidden_size, expert_ffn, E, int(nthreads))
    if rc != 0:
        raise ValueError(f"chimere_ncmoe_experts rejected its arguments (code {rc})")
    return out
