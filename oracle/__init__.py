"""CPU oracle for the quantized decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package, and only as the checker.  It wraps ``liboracle.so``
(built from oracle.c by oracle/Makefile) with numpy-facing helpers.
"""
import ctypes as _C
import os as _os
import subprocess as _sp

import numpy as np

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ3_S, MXFP4 = 2, 8, 12, 13, 14, 21, 39
Q4_0_SFORM = 102   # not a ggml type: Q4_0 blocks with ggml's s-form block term (gemv only)
_HERE = _os.path.dirname(_os.path.abspath(__file__))
_LIB = None


def build():
    _sp.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = _os.path.join(_HERE, "liboracle.so")
        if not _os.path.exists(path):
            build()
        L = _C.CDLL(path)
        vp, i64, i32, f32 = _C.c_void_p, _C.c_int64, _C.c_int, _C.c_float
        L.orc_f32_to_f16.restype = _C.c_uint16
        L.orc_f32_to_f16.argtypes = [f32]
        L.orc_f16_to_f32.restype = f32
        L.orc_f16_to_f32.argtypes = [_C.c_uint16]
        L.orc_exp.restype = f32
        L.orc_exp.argtypes = [f32]
        L.orc_silu.restype = f32
        L.orc_silu.argtypes = [f32]
        L.orc_row_bytes.restype = i64
        L.orc_row_bytes.argtypes = [i32, i64]
        L.orc_quantize_q8_1.argtypes = [vp, i64, i64, i64, vp]
        for n in ("orc_quantize_q8_0", "orc_quantize_q4_0", "orc_quantize_iq3_s"):
            getattr(L, n).argtypes = [vp, i64, vp]
        L.orc_dequantize.argtypes = [i32, vp, i64, vp]
        L.orc_block_dots.argtypes = [i32, vp, vp, i32, i32, vp]
        L.orc_gemv.argtypes = [i32, vp, vp, i64, vp, i32, i32, i32, i32, i32, i32]
        L.orc_gemv_q8_0_f64.argtypes = [vp, vp, vp, i32, i32]
        L.orc_router.argtypes = [vp, vp, vp, i32, i32]
        L.orc_topk_softmax.argtypes = [vp, i32, i32, vp, vp]
        L.orc_moe.argtypes = [vp, vp, vp, vp, vp, i32]
        L.cpb_gemv.argtypes = [i32, vp, vp, vp, i32, i32, i32]
        L.cpb_moe.argtypes = [vp, vp, vp, vp, vp, i32]
        L.orc_fused_moe_iq3s.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, i64, i64, i64, i32]
        L.orc_quantize_q8_K.argtypes = [vp, i64, vp]
        L.orc_vec_dot_iq3s_q8K.restype = f32
        L.orc_vec_dot_iq3s_q8K.argtypes = [i32, vp, vp]
        L.orc_gemv_iq3s_q8K.argtypes = [vp, vp, vp, i32, i32]
        L.orc_moe_ncmoe.argtypes = [vp, vp, vp, vp, vp, i32]
        L.orc_ncmoe.argtypes = [vp, vp, vp, i64, i64, i64, vp, vp, i32, vp, vp, i32, i32]
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(_C.c_void_p) if a is not None else None


def pad512(n):
    return (n + 511) // 512 * 512


def row_bytes(t, ncols):
    return {Q8_0: ncols // 32 * 34, Q4_0: ncols // 32 * 18, Q4_0_SFORM: ncols // 32 * 18, IQ3_S: ncols // 256 * 110,
            Q4_K: ncols // 256 * 144,
            Q5_K: ncols // 256 * 176, Q6_K: ncols // 256 * 210, MXFP4: ncols // 32 * 17}[t]


def f32_to_f16(x):
    return lib().orc_f32_to_f16(float(x))


def f16_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def exp(x):
    return lib().orc_exp(float(x))


def silu(x):
    return lib().orc_silu(float(x))


def quantize_q8_1(x, ncols_padded=None):
    """x: [nrows, ncols] or [ncols] f32 -> uint8 [nrows, ncols_padded/32*36]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    ncols = x2.shape[1]
    ncp = ncols_padded or pad512(ncols)
    out = np.zeros((x2.shape[0], ncp // 32 * 36), np.uint8)
    lib().orc_quantize_q8_1(_p(x2), ncols, ncp, x2.shape[0], _p(out))
    return out if x.ndim > 1 else out[0]


def quantize(t, x):
    """Weight quantizer for type t; x [..., ncols] f32 -> uint8 rows."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    out = np.zeros(n // (256 if t == IQ3_S else 32) * (110 if t == IQ3_S else (34 if t == Q8_0 else 18)), np.uint8)
    fn = {Q8_0: "orc_quantize_q8_0", Q4_0: "orc_quantize_q4_0", IQ3_S: "orc_quantize_iq3_s"}[t]
    getattr(lib(), fn)(_p(x), n, _p(out))
    if x.ndim > 1:
        out = out.reshape(x.shape[:-1] + (row_bytes(t, x.shape[-1]),))
    return out


def dequantize(t, w, n):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.zeros(n, np.float32)
    lib().orc_dequantize(t, _p(w), n, _p(out))
    return out


def block_dots(t, W, xq, ncols, nrows):
    out = np.zeros((nrows, ncols // 32), np.int32)
    lib().orc_block_dots(t, _p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(xq)), ncols, nrows, _p(out))
    return out


def gemv(t, W, xq, ncols, nrows, L=16, G=1, ntok=1, xq_stride=0, nthreads=0):
    y = np.zeros((ntok, nrows), np.float32)
    lib().orc_gemv(t, _p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(xq)), xq_stride,
                   _p(y), ncols, nrows, ntok, L, G, nthreads)
    return y[0] if ntok == 1 else y


def gemv_q8_0_f64(W, x, ncols, nrows):
    y = np.zeros(nrows, np.float32)
    lib().orc_gemv_q8_0_f64(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(x, np.float32)), _p(y), ncols, nrows)
    return y


def fused_moe_iq3s(x, gate, up, down, ids, wts, out, H, F, bg, bu, bd):
    """out (f32 [H], updated in place) += the f32-activation IQ3_S expert FFN of the
    experts ids with weights wts (the library's fixed order)."""
    ids = np.ascontiguousarray(ids, np.int32)
    lib().orc_fused_moe_iq3s(_p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(gate)),
                             _p(np.ascontiguousarray(up)), _p(np.ascontiguousarray(down)), _p(ids),
                             _p(np.ascontiguousarray(wts, np.float32)), _p(out), H, F, bg, bu, bd, ids.size)
    return out


def router(Wr, x):
    E, H = Wr.shape
    out = np.zeros(E, np.float32)
    lib().orc_router(_p(np.ascontiguousarray(Wr, np.float32)), _p(np.ascontiguousarray(x, np.float32)), _p(out), E, H)
    return out


def topk_softmax(logits, K):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.zeros(K, np.int32)
    w = np.zeros(K, np.float32)
    lib().orc_topk_softmax(_p(logits), logits.size, K, _p(idx), _p(w))
    return idx, w


class _MoeParams(_C.Structure):
    _fields_ = [("H", _C.c_int), ("F", _C.c_int), ("E", _C.c_int), ("K", _C.c_int), ("M", _C.c_int),
                ("exp_type", _C.c_int), ("sh_type", _C.c_int),
                ("router", _C.c_void_p), ("logit_bias", _C.c_void_p),
                ("gate", _C.c_void_p), ("up", _C.c_void_p), ("down", _C.c_void_p),
                ("stride_gate", _C.c_int64), ("stride_up", _C.c_int64), ("stride_down", _C.c_int64),
                ("sh_gate", _C.c_void_p), ("sh_up", _C.c_void_p), ("sh_down", _C.c_void_p),
                ("sh_gate_w", _C.c_void_p), ("L", _C.c_int), ("G", _C.c_int)]


def moe(x, router_w, gate, up, down, exp_type, K, sh=None, sh_type=-1, sh_gate_w=None,
        logit_bias=None, L=16, G=1, nthreads=0, fn="orc_moe"):
    """MoE FFN for x [M, H]; gate/up [E, F*rowbytes(H)] down [E, H*rowbytes(F)]
    (uint8, one row per expert).  sh = (gate, up, down) or None.
    Returns (out [M,H], ids [M,K], wts [M,K])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, router_w.shape[1])
    M, H = x.shape
    E = router_w.shape[0]
    F = gate.size // E // row_bytes(exp_type, H)
    keep = [np.ascontiguousarray(a) if a is not None else None
            for a in (router_w.astype(np.float32), gate, up, down, logit_bias, sh_gate_w)]
    shk = [np.ascontiguousarray(a) for a in sh] if sh is not None else [None, None, None]
    p = _MoeParams(H, F, E, K, M, exp_type, sh_type if sh is not None else -1,
                   _p(keep[0]), _p(None if logit_bias is None else keep[4].astype(np.float32)),
                   _p(keep[1]), _p(keep[2]), _p(keep[3]),
                   gate.size // E, up.size // E, down.size // E,
                   _p(shk[0]), _p(shk[1]), _p(shk[2]),
                   _p(None if sh_gate_w is None else keep[5]), L, G)
    lb = None if logit_bias is None else np.ascontiguousarray(logit_bias, np.float32)
    if lb is not None:
        p.logit_bias = _p(lb)
    if sh_gate_w is not None:
        sgw = np.ascontiguousarray(sh_gate_w, np.float32)
        p.sh_gate_w = _p(sgw)
    out = np.zeros((M, H), np.float32)
    ids = np.zeros((M, K), np.int32)
    wts = np.zeros((M, K), np.float32)
    getattr(lib(), fn)(_C.byref(p), _p(x), _p(out), _p(ids), _p(wts), nthreads)
    return out, ids, wts


def moe_ncmoe(*args, **kw):
    """moe() with the routed experts on the ncmoe CPU path (Q8_K activations,
    IQ3_S experts); router, top-k and shared expert as moe()."""
    return moe(*args, fn="orc_moe_ncmoe", **kw)


def cpu_moe(*args, nthreads=1, **kw):
    """The CPU baseline (cpu_path.c): same arguments and results as moe(),
    to the fp32 tolerance."""
    return moe(*args, nthreads=nthreads, fn="cpb_moe", **kw)


def cpu_gemv(t, W, xq, ncols, nrows, nthreads=1):
    """CPU baseline GEMV of one Q8_1 row (cpu_path.c)."""
    y = np.zeros(nrows, np.float32)
    lib().cpb_gemv(t, _p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(xq)), _p(y), ncols, nrows, nthreads)
    return y


def quantize_q8_K(x):
    """ggml Q8_K blocks (296 B per 256 values) of a float vector."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    assert x.size % 256 == 0
    out = np.zeros(x.size // 256 * 296, np.uint8)
    lib().orc_quantize_q8_K(_p(x), x.size, _p(out))
    return out


def vec_dot_iq3s_q8K(w, y, n):
    return lib().orc_vec_dot_iq3s_q8K(int(n), _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(y)))


def gemv_iq3s_q8K(W, x, nrows, ncols):
    """y = W x, IQ3_S rows against the Q8_K quantization of f32 x."""
    W = np.ascontiguousarray(W, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(nrows, np.float32)
    lib().orc_gemv_iq3s_q8K(_p(W), _p(x), _p(y), nrows, ncols)
    return y


def ncmoe(x, gate, up, down, ids, wts, H, F):
    """The CPU expert loop of one token: sum_k w_k * down_e(silu(gate_e x) * up_e x)
    with IQ3_S expert tensors [E, rows * row_bytes]."""
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    ids = np.ascontiguousarray(ids, np.int32)
    wts = np.ascontiguousarray(wts, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(H, np.float32)
    sg, su, sd = (a[0].size if a.ndim == 2 else a.size // 256 for a in (gate, up, down))
    lib().orc_ncmoe(_p(gate), _p(up), _p(down), sg, su, sd, _p(ids), _p(wts), ids.size, _p(x), _p(out), H, F)
    return out
