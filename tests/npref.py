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
