"""Independent numpy restatement of the block formats, used to cross-check the
C oracle (the two are written separately, so a slip in one shows up as a
mismatch).  Layouts follow chimere-server/src/gguf_loader.rs:752-772 (Q4_0),
:793-837 (Q8_0), :1008-1142 (IQ3_S) and the Q8_1 layout of
kernels/chimere_kernels.cu:1495-1523."""
import json
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def load_grid(path=None):
    path = path or os.path.join(ROOT, "chimere_amd", "csrc", "iq3s_grid.inc")
    txt = open(path).read()
    return np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", txt)], dtype=np.uint32)


GRID = load_grid()


def f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def levels(t, W, ncols):
    """Integer levels [nrows, ncols] (int64) and per-32-block f32 scale [nrows, ncols/32]."""
    W = np.asarray(W, np.uint8).reshape(-1, {8: ncols // 32 * 34, 2: ncols // 32 * 18, 21: ncols // 256 * 110}[t])
    R = W.shape[0]
    if t == 8:
        B = W.reshape(R, ncols // 32, 34)
        d = f16(B[:, :, 0].astype(np.uint16) | (B[:, :, 1].astype(np.uint16) << 8))
        q = B[:, :, 2:].view(np.int8).astype(np.int64).reshape(R, ncols)
        return q, d
    if t == 2:
        B = W.reshape(R, ncols // 32, 18)
        d = f16(B[:, :, 0].astype(np.uint16) | (B[:, :, 1].astype(np.uint16) << 8))
        qs = B[:, :, 2:].astype(np.int64)
        q = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=2).reshape(R, ncols)
        return q, d
    B = W.reshape(R, ncols // 256, 110)
    d = f16(B[:, :, 0].astype(np.uint16) | (B[:, :, 1].astype(np.uint16) << 8))
    q = np.zeros((R, ncols // 256, 8, 32), np.int64)
    mult = np.zeros((R, ncols // 256, 8), np.int64)
    for ib in range(8):
        sc = (B[:, :, 106 + ib // 2].astype(np.int64) >> (4 * (ib & 1))) & 15
        mult[:, :, ib] = 1 + 2 * sc
        qh = B[:, :, 66 + ib].astype(np.int64)
        for l in range(4):
            sg = B[:, :, 74 + 4 * ib + l].astype(np.int64)
            for h in range(2):
                idx = B[:, :, 2 + 8 * ib + 2 * l + h].astype(np.int64) | (((qh >> (2 * l + h)) & 1) << 8)
                gv = GRID[idx].astype(np.int64)
                for j in range(4):
                    lv = (gv >> (8 * j)) & 255
                    neg = (sg >> (4 * h + j)) & 1
                    q[:, :, ib, 8 * l + 4 * h + j] = np.where(neg == 1, -lv, lv)
    q = q * mult[..., None]
    dd = np.repeat(d, 8, axis=1)
    return q.reshape(R, ncols), dd


def dequant(t, W, ncols):
    q, d = levels(t, W, ncols)
    return (q.reshape(q.shape[0], -1, 32) * d[..., None].astype(np.float64)).reshape(q.shape[0], ncols)


def q8_1_fields(xq, nblocks):
    B = np.asarray(xq, np.uint8).reshape(-1, 36)[:nblocks]
    d = f16(B[:, 0].astype(np.uint16) | (B[:, 1].astype(np.uint16) << 8))
    s = f16(B[:, 2].astype(np.uint16) | (B[:, 3].astype(np.uint16) << 8))
    q = B[:, 4:].view(np.int8).astype(np.int64)
    return d, s, q


def block_dots(t, W, xq, ncols):
    q, _ = levels(t, W, ncols)
    _, _, qx = q8_1_fields(xq, ncols // 32)
    return (q.reshape(q.shape[0], -1, 32) * qx[None]).sum(-1)


def gemv_f64(t, W, xq, ncols):
    """y = sum_b d_w d_x sumi_b in float64 (order-free reference)."""
    q, dw = levels(t, W, ncols)
    dx, _, qx = q8_1_fields(xq, ncols // 32)
    s = (q.reshape(q.shape[0], -1, 32) * qx[None]).sum(-1).astype(np.float64)
    return (s * dw.astype(np.float64) * dx.astype(np.float64)[None]).sum(-1)


# ---- ggml K-quants and MXFP4, restated per the reference's dequantizers
# (gguf_loader.rs:839-917 Q6_K, :1165-1263 Q5_K, :1265-1330 Q4_K: groups of
# 64 elements for Q4_K/Q5_K, of 128 for Q6_K) and ggml's MXFP4 layout.

KQ_BYTES = {12: 144, 13: 176, 14: 210, 39: 17}


def _scale_min(sc12, j):
    """get_scale_min_k4 (gguf_loader.rs:1150-1163) on [..., 12] uint8 arrays."""
    s = sc12.astype(np.int64)
    if j < 4:
        return s[..., j] & 63, s[..., j + 4] & 63
    return (s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4), (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)


def kq_parts(t, W, ncols):
    """Integer quants q [R, ncols] and per-32-block (d*sc, dmin*m) factors as
    float64 pairs (scale [R, ncols/32], minv [R, ncols/32]) such that
    w = scale * q - minv (Q6_K: q already signed, minv 0, scale per 16
    elements collapsed per half via q*sc; MXFP4: q the doubled E2M1 level)."""
    R = np.asarray(W).size // (ncols // (32 if t == 39 else 256) * KQ_BYTES[t])
    if t == 39:
        B = np.asarray(W, np.uint8).reshape(R, ncols // 32, 17)
        e = B[:, :, 0].astype(np.int64)
        lv = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.int64)
        qs = B[:, :, 1:].astype(np.int64)
        q = np.concatenate([lv[qs & 15], lv[qs >> 4]], axis=2).reshape(R, ncols)
        return q, np.ldexp(1.0, e - 128), np.zeros(e.shape)
    nsb = ncols // 256
    B = np.asarray(W, np.uint8).reshape(R, nsb, KQ_BYTES[t])
    q = np.zeros((R, nsb, 256), np.int64)
    scale = np.zeros((R, nsb, 8), np.float64)
    minv = np.zeros((R, nsb, 8), np.float64)
    if t in (12, 13):
        d = f16(B[:, :, 0].astype(np.uint16) | (B[:, :, 1].astype(np.uint16) << 8)).astype(np.float64)
        dmin = f16(B[:, :, 2].astype(np.uint16) | (B[:, :, 3].astype(np.uint16) << 8)).astype(np.float64)
        qs0 = 16 if t == 12 else 48
        for g in range(4):                       # 64-element groups, sub-blocks 2g, 2g+1
            ql = B[:, :, qs0 + 32 * g: qs0 + 32 * g + 32].astype(np.int64)
            lo, hi = ql & 15, ql >> 4
            if t == 13:
                qh = B[:, :, 16:48].astype(np.int64)
                lo = lo + 16 * ((qh >> (2 * g)) & 1)
                hi = hi + 16 * ((qh >> (2 * g + 1)) & 1)
            q[:, :, 64 * g: 64 * g + 32] = lo
            q[:, :, 64 * g + 32: 64 * g + 64] = hi
            for k in range(2):
                sc, m = _scale_min(B[:, :, 4:16], 2 * g + k)
                scale[:, :, 2 * g + k] = d * sc
                minv[:, :, 2 * g + k] = dmin * m
        return q.reshape(R, ncols), scale.reshape(R, -1), minv.reshape(R, -1)
    # Q6_K
    d = f16(B[:, :, 208].astype(np.uint16) | (B[:, :, 209].astype(np.uint16) << 8)).astype(np.float64)
    sc = B[:, :, 192:208].view(np.int8).astype(np.int64)
    for g in range(2):                           # 128-element groups
        ql = B[:, :, 64 * g: 64 * g + 64].astype(np.int64)
        qh = B[:, :, 128 + 32 * g: 160 + 32 * g].astype(np.int64)
        base = 128 * g
        q[:, :, base: base + 32] = (ql[:, :, :32] & 15) | (((qh >> 0) & 3) << 4)
        q[:, :, base + 32: base + 64] = (ql[:, :, 32:] & 15) | (((qh >> 2) & 3) << 4)
        q[:, :, base + 64: base + 96] = (ql[:, :, :32] >> 4) | (((qh >> 4) & 3) << 4)
        q[:, :, base + 96: base + 128] = (ql[:, :, 32:] >> 4) | (((qh >> 6) & 3) << 4)
    q = (q - 32) * np.repeat(sc, 16, axis=2)     # scale per 16 elements folded into q
    scale[:] = d[:, :, None]
    return q.reshape(R, ncols), scale.reshape(R, -1), minv.reshape(R, -1)


def kq_dequant(t, W, ncols):
    q, scale, minv = kq_parts(t, W, ncols)
    R = q.shape[0]
    return (q.reshape(R, -1, 32) * scale[..., None] - minv[..., None]).reshape(R, ncols)


def kq_gemv_f64(t, W, xq, ncols):
    """Order-free float64 reference: sum_i w_i * d_x * q_x (w from kq_dequant)."""
    dx, _, qx = q8_1_fields(xq, ncols // 32)
    xd = (qx.astype(np.float64) * dx.astype(np.float64)[:, None]).reshape(-1)
    return kq_dequant(t, W, ncols) @ xd


def kq_block_dots(t, W, xq, ncols):
    """The debug entry point's int32: sc*sum(q*q_x) (Q4_K/Q5_K), sum((q-32)*sc*q_x)
    (Q6_K), sum(level*q_x) (MXFP4)."""
    q, _, _ = kq_parts(t, W, ncols)
    R = q.shape[0]
    _, _, qx = q8_1_fields(xq, ncols // 32)
    s = (q.reshape(R, -1, 32) * qx[None]).sum(-1)
    if t in (12, 13):
        B = np.asarray(W, np.uint8).reshape(R, ncols // 256, KQ_BYTES[t])
        sc = np.stack([_scale_min(B[:, :, 4:16], j)[0] for j in range(8)], axis=2).reshape(R, -1)
        s = s * sc
    return s


# ---- independent packers (ggml's quantizer-side field packing), used to
# pin the readers above and the oracle on crafted blocks.

def pack_kq_scales(sc, m):
    """8 six-bit scales and mins -> 12 bytes (the inverse of get_scale_min_k4)."""
    out = np.zeros(12, np.uint8)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return out


def pack_q4_k(d16, dmin16, sc, m, q):
    """q: 256 ints 0..15; element 64g + l (l<32) -> low nibble of qs[32g + l],
    64g + 32 + l -> high nibble."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d16], np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin16], np.uint16).view(np.uint8)
    b[4:16] = pack_kq_scales(sc, m)
    for g in range(4):
        for l in range(32):
            b[16 + 32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    return b


def pack_q5_k(d16, dmin16, sc, m, q):
    """q: 256 ints 0..31; bit 4 of element 32j + l goes to bit j of qh[l]."""
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([d16], np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin16], np.uint16).view(np.uint8)
    b[4:16] = pack_kq_scales(sc, m)
    for j in range(8):
        for l in range(32):
            b[16 + l] |= ((q[32 * j + l] >> 4) & 1) << j
    for g in range(4):
        for l in range(32):
            b[48 + 32 * g + l] = (q[64 * g + l] & 15) | ((q[64 * g + 32 + l] & 15) << 4)
    return b


def pack_q6_k(d16, sc16, q):
    """q: 256 ints 0..63 (value q-32); ggml's quantize_row_q6_K packing per
    128-element half h: ql[64h + l] = q[l] | q[64 + l] << 4, ql[64h + 32 + l]
    = q[32 + l] | q[96 + l] << 4, qh[32h + l] = the four high pairs."""
    b = np.zeros(210, np.uint8)
    for h in range(2):
        Q = q[128 * h: 128 * h + 128]
        for l in range(32):
            b[64 * h + l] = (Q[l] & 15) | ((Q[64 + l] & 15) << 4)
            b[64 * h + 32 + l] = (Q[32 + l] & 15) | ((Q[96 + l] & 15) << 4)
            b[128 + 32 * h + l] = (Q[l] >> 4) | ((Q[32 + l] >> 4) << 2) | ((Q[64 + l] >> 4) << 4) | ((Q[96 + l] >> 4) << 6)
    b[192:208] = np.asarray(sc16, np.int8).view(np.uint8)
    b[208:210] = np.array([d16], np.uint16).view(np.uint8)
    return b


def rand_kq(t, nrows, ncols, rng):
    """Random valid blocks of a K-quant / MXFP4 type: random quant and scale
    bytes, finite f16 super-scales (d ~ 1e-3, dmin ~ 2e-4), E8M0 bytes near 2^-6."""
    n = ncols // (32 if t == 39 else 256)
    B = rng.integers(0, 256, (nrows, n, KQ_BYTES[t]), dtype=np.uint8)
    h = lambda v: np.asarray(v, np.float16).view(np.uint16)
    if t in (12, 13):
        B[:, :, 0:2] = h(rng.uniform(0.5e-3, 1.5e-3, (nrows, n))).view(np.uint8).reshape(nrows, n, 2)
        B[:, :, 2:4] = h(rng.uniform(0.5e-4, 3e-4, (nrows, n))).view(np.uint8).reshape(nrows, n, 2)
    elif t == 14:
        B[:, :, 208:210] = h(rng.uniform(0.5e-4, 1.5e-4, (nrows, n))).view(np.uint8).reshape(nrows, n, 2)
    else:
        B[:, :, 0] = rng.integers(118, 124, (nrows, n))
    return B.reshape(nrows, -1)
