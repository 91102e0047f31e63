"""Host-side emulation of the index arithmetic of the one-token MoE kernels
(k_moe_route<1>, k_moe_expert1 with its helper prefetch, k_moe_dc1 in
chimere_amd/csrc/moe.hip), at the shapes of the one-token tie tests and of
the model: every global byte range and LDS index each thread forms is
computed here, vectorised over threads, and checked against the size of the
allocation it addresses.  The formulas are transcribed from the kernels and
launch code (grid sizes, item mapping, chunk copies, prefetch ranges, plan /
weight / Q8_1 writes, down-row reads); a slip that sends an index out of its
array on some (work-group, thread) fails here, on the CPU.

Routing is the one input the indices depend on: every case is run with the
selected experts at the lowest ids, at the highest ids, and spread, so the
(expert * stride) terms reach both ends of the stacked tensors."""
import numpy as np
import pytest

QK, SLOTS, Q8_1 = 32, 16, 36
EX_THREADS = 1024
E1_ROWS = 2 * QK // (EX_THREADS // 64)
DC1_ROWS = 4
E1_MAX_H = 2048
ROW_PAD = 512
BYTES = {"q4_0": 18, "q8_0": 34}
PLAN_UEXP = 1
PLAN_INTS = 1 + 2 * 8 * 16 + 8 * 16 * 8 + 1 + 4 * 8 * 16


def row_bytes(t, n):
    return n // QK * BYTES[t]


def e1_cblk(t):
    return 16 if t == "q8_0" else 32


def chunk_bytes(t, blocks):
    return blocks * BYTES[t]


class Checker:
    def __init__(self):
        self.n = 0

    def rng(self, what, lo, hi, size):
        """Byte range [lo, hi) (arrays) inside [0, size)."""
        lo, hi = np.asarray(lo), np.asarray(hi)
        self.n += lo.size
        assert (lo >= 0).all() and (hi <= size).all(), \
            f"{what}: range [{lo.min()}, {hi.max()}) outside [0, {size})"


def emulate(H, F, E, K, te, ts, has_shared, ids, grid=256):
    """All index checks of one layer call; returns the number of ranges checked."""
    ck = Checker()
    NB, nbH = F // QK, H // QK
    rbH_e, rbH_s = row_bytes(te, H), row_bytes(ts, H)
    rbF_e, rbF_s = row_bytes(te, F), row_bytes(ts, F)
    gate_sz = E * F * rbH_e            # stacked gate (= up) tensor bytes, stride F * rbH
    down_sz = E * H * rbF_e
    sd = H * rbF_e
    shg_sz, shd_sz = F * rbH_s, H * rbF_s
    xq_stride = (H + ROW_PAD - 1) // ROW_PAD * ROW_PAD // QK * Q8_1
    hq_stride = (F + ROW_PAD - 1) // ROW_PAD * ROW_PAD // QK * Q8_1
    P = K + 1
    t = np.arange(EX_THREADS)
    wave, lane = t >> 6, t & 63
    # ---- K1 k_moe_route<1>: grid E + ng + ceil(nbH / 8) (no shared gate row here)
    nq = (nbH + 7) // 8
    for row in range(E + nq):
        if row >= E:
            b0 = (row - E) * 8
            nblk = min(8, nbH - b0)
            ck.rng("route: x read", b0 * QK * 4, (b0 + nblk) * QK * 4, H * 4)
            ck.rng("route: xq write", b0 * Q8_1, (b0 + nblk) * Q8_1, xq_stride)
        else:
            ck.rng("route: router row", row * H * 4, (row + 1) * H * 4, E * H * 4)
            ck.rng("route: logits", row * 4, row * 4 + 4, E * 4)
    # ---- K2 k_moe_expert1: grid = min(items, CUs) = 256 here
    CB = max(e1_cblk(te) * BYTES[te], e1_cblk(ts) * BYTES[ts] if has_shared else 0)
    buf_sz = 2 * QK * CB + 16                  # bufA / bufB: 64 chunk rows + 16 bytes of slack
    ns_tot = (NB + 7) // 8 if has_shared else 0
    assert NB + ns_tot <= grid // 8          # expert1_fits
    for b in range(grid):
        x, lb, G8 = b & 7, b >> 3, grid >> 3
        nr = 1 if K > x else 0
        ns = ((NB - 1 - x) // 8 + 1 if NB > x else 0) if has_shared else 0
        nx = nr * NB + ns
        routed = lb < nr * NB
        shared = (not routed) and lb < nx
        # Q8_1(x) decode into xs[E1_MAX_H / QK] (waves 1.. of routed, all threads of shared)
        i = t - 64 if routed else t
        act = (i >= 0) & (i < nbH)
        ck.rng("expert1: xs index", i[act] * 40, i[act] * 40 + 40, E1_MAX_H // QK * 40)
        ck.rng("expert1: xq read", i[act] * Q8_1, i[act] * Q8_1 + Q8_1, xq_stride)
        if not shared:
            if b == 0:
                ck.rng("expert1: wts/plan", (PLAN_UEXP + t[t < K]) * 4, (PLAN_UEXP + t[t < K]) * 4 + 4, PLAN_INTS * 4)
            if not routed:
                # helper: e1_prefetch of rows [x H/8, (x+1) H/8) of every pair's down matrix
                nh, hb = G8 - nx, lb - nx
                mb, sb = H * rbF_e, H * rbF_s
                sE, sS = mb // 8, sb // 8
                total = K * sE + (sS if has_shared else 0)
                lo, hi = total * hb // nh, total * (hb + 1) // nh
                o0 = lo + 64 * t
                os_ = [o0 + 64 * EX_THREADS * s for s in range(int((hi - lo) // (64 * EX_THREADS)) + 2)]
                o = np.concatenate(os_)
                o = o[o < hi]
                m = o // sE
                rt = m < K
                off_r = ids[m[rt]] * sd + x * sE + ((o[rt] - m[rt] * sE) & ~1)
                ck.rng("expert1: prefetch routed down", off_r, off_r + 2, down_sz)
                off_s = x * sS + ((o[~rt] - K * sE) & ~1)
                if off_s.size:
                    assert has_shared
                    ck.rng("expert1: prefetch shared down", off_s, off_s + 2, shd_sz)
                continue
            e, pair, w, T, rb = ids[x], x, lb, te, rbH_e
            base_sz, base_off = gate_sz, e * F * rbH_e
        else:
            pair, w, T, rb = K, x + 8 * (lb - nr * NB), ts, rbH_s
            base_sz, base_off = shg_sz, 0
        assert w < NB, "item block w out of range"
        # e1_item: chunks of the 2*QK rows [32w, 32w+32) of gate and up
        cblk = e1_cblk(T)
        nc = (nbH + cblk - 1) // cblk
        for c in range(nc):
            cb = min(cblk, nbH - c * cblk)
            goff = chunk_bytes(T, c * cblk)
            pre = goff & 15
            span = pre + chunk_bytes(T, cb)
            for k in range(E1_ROWS):
                r = wave + (EX_THREADS // 64) * k
                a = lane * 16 < span
                src = base_off + (w * QK + (r % QK)) * rb + goff - pre + lane * 16
                ck.rng("expert1: gate/up copy", src[a], src[a] + 16, base_sz)
                dst = r * CB + lane * 16
                ck.rng("expert1: LDS chunk", dst[a], dst[a] + 16, buf_sz - 16)
            # e1_dots reads: row g, blocks j, j+16, ... < cb (lds_u32 needs 4 bytes slack)
            g, j = t >> 4, t & 15
            for bb in range(0, cblk, SLOTS):
                blk = j + bb
                a = blk < cb
                lo_ = g * CB + pre + blk * BYTES[T]
                ck.rng("expert1: LDS dot", lo_[a], lo_[a] + BYTES[T] + 4, buf_sz)
                ck.rng("expert1: xs dot", (c * cblk + blk[a]) * 40, (c * cblk + blk[a]) * 40 + 40,
                       E1_MAX_H // QK * 40)
        # Q8_1(h) block w of `pair`: half-wave 0
        o = pair * hq_stride + w * Q8_1
        ck.rng("expert1: hq write", o, o + Q8_1, P * hq_stride)
    # ---- K3 k_moe_dc1: grid H / 4, (K + has_shared + 1) * 64 threads (the
    # last wave loads the routing weights and the gate logit into LDS)
    G3 = H // DC1_ROWS
    assert G3 % 8 == 0
    npair = K + int(has_shared)
    nthr = (npair + 1) * 64
    assert nthr <= 1024
    t3 = np.arange(nthr)
    j, rr, p = t3 & 15, (t3 >> 4) & (DC1_ROWS - 1), t3 >> 6
    lane = t3 & 63
    ld = (p == npair) & (lane < K)
    ck.rng("dc1: wts read", lane[ld] * 4, lane[ld] * 4 + 4, K * 4)
    ck.rng("dc1: s_wk write", lane[ld] * 4, lane[ld] * 4 + 4, 9 * 4)
    if has_shared:
        ck.rng("dc1: s_wk gate logit", np.array([K * 4]), np.array([K * 4 + 4]), 9 * 4)
    for b in range(G3):
        tile_i = (b & 7) * (G3 >> 3) + (b >> 3)
        assert tile_i < G3
        r = tile_i * DC1_ROWS + rr
        act = (j < NB) & (r < H) & (p < npair)
        hb = p * hq_stride + j * Q8_1
        ck.rng("dc1: hq read", hb[act], hb[act] + Q8_1, P * hq_stride)
        rt = act & (p < K)
        ck.rng("dc1: plan read", (PLAN_UEXP + p[rt]) * 4, (PLAN_UEXP + p[rt]) * 4 + 4, PLAN_INTS * 4)
        off = ids[p[rt]] * sd + r[rt] * rbF_e + j[rt] * BYTES[te]
        ck.rng("dc1: routed down row", off, off + BYTES[te], down_sz)
        sh = act & (p == K)
        off = r[sh] * rbF_s + j[sh] * BYTES[ts]
        ck.rng("dc1: shared down row", off, off + BYTES[ts], shd_sz)
        wr = (j == 0) & (p < npair)
        ck.rng("dc1: dn LDS", (rr[wr] * 9 + p[wr]) * 4, (rr[wr] * 9 + p[wr]) * 4 + 4, DC1_ROWS * 9 * 4)
        ck.rng("dc1: out", (tile_i * DC1_ROWS + np.arange(DC1_ROWS)) * 4,
               (tile_i * DC1_ROWS + np.arange(DC1_ROWS)) * 4 + 4, H * 4)
    return ck.n


CASES = [
    # the two one-token tie tests held off the GPU, and the model's shapes
    ("zero-input tie", 1024, 256, 32, 4, "q4_0", "q4_0", True),
    ("pair-tied rows", 1024, 256, 64, 7, "q4_0", "q4_0", True),
    ("config 3", 2048, 512, 256, 8, "q4_0", "q4_0", True),
    ("q8_0 model shape", 2048, 512, 256, 8, "q8_0", "q8_0", True),
    ("mixed, one K chunk", 256, 256, 16, 3, "q8_0", "q4_0", True),
    ("no shared", 2048, 512, 64, 8, "q4_0", "q4_0", False),
]


@pytest.mark.parametrize("name,H,F,E,K,te,ts,sh", CASES)
def test_one_token_kernel_indices_in_bounds(name, H, F, E, K, te, ts, sh):
    rng = np.random.default_rng(H + E + K)
    for ids in (np.arange(K), np.arange(E - K, E), np.sort(rng.choice(E, K, replace=False))):
        assert emulate(H, F, E, K, te, ts, sh, np.asarray(ids, np.int64)) > 0


def test_checker_catches_an_overrun():
    """The emulation would flag a slip: a helper range one 64-byte step too long."""
    ck = Checker()
    with pytest.raises(AssertionError):
        ck.rng("probe", np.array([0]), np.array([1025]), 1024)
