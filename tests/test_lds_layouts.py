"""Host-side check of the padded LDS row layouts of the asynchronous copies:

* stage_rows with an LDS row stride above the row bytes (chimere_amd/csrc/
  common.h), as the GEMV tile uses it (chimere_amd/csrc/tile_gemv.h,
  mmvq.hip: Q4_0 / Q8_0 / IQ3_S chunks, row padding 48 / 48 / 80 bytes);
* the two-stage prefill copy loop (chimere_amd/csrc/prefill.hip, pf_gemm_k):
  weight rows in slots of pf_lds_row_al bytes (IQ3_S 128 -> 144) and the
  tile's activation rows in slots of 304 bytes (8 Q8_1 blocks + 16).

The slot -> (row, column) arithmetic is transcribed from the kernels.  Every
16-byte piece of every row must be written exactly once, no write may leave
its LDS buffer, no padding slot may be written, and the readers' furthest
byte (last block of the last row, plus the 4 bytes an unaligned 32-bit LDS
read may touch) must stay inside the buffer."""
import pytest

QK = 32
BYTES = {"q4_0": 18, "q8_0": 34, "iq3s": 110, "q6k": 210}
ELEMS = {"q4_0": 32, "q8_0": 32, "iq3s": 256, "q6k": 256}


def chunk_bytes(t, blocks):
    return blocks * QK // ELEMS[t] * BYTES[t]


def stage_rows_padded(nrows, seg, lseg, gstride, nthreads):
    """(lds byte offset, global byte offset) of every piece the padded path copies."""
    per, lper = seg // 16, lseg // 16
    tot = lper * nrows
    out = []
    for wave in range(nthreads // 64):
        for c0 in range(wave * 64, tot, (nthreads // 64) * 64):
            for lane in range(64):
                c = c0 + lane
                r, col = divmod(c, lper)
                if c < tot and col < per:
                    out.append((c0 * 16 + lane * 16, r * gstride + col * 16, r, col))
    return out


@pytest.mark.parametrize("t,pad", [("q4_0", 48), ("q8_0", 48), ("iq3s", 80)])
@pytest.mark.parametrize("ncols", [2048, 4096, 2048 + 512, 256 * 3])
def test_gemv_tile_padded_rows(t, pad, ncols):
    TILE_ROWS, CBLK, NTH = 16, 64, 256
    CB = chunk_bytes(t, CBLK)
    buf = TILE_ROWS * (CB + pad) + 16
    rb = ncols // ELEMS[t] * BYTES[t]
    nb = ncols // QK
    for b0 in range(0, nb, CBLK):
        cb = min(CBLK, nb - b0)
        seg = chunk_bytes(t, cb)
        goff = b0 * QK // ELEMS[t] * BYTES[t]
        padded = (seg | goff) % 16 == 0 and rb % 16 == 0
        if not padded:
            continue
        lseg = seg + pad
        for nr in (TILE_ROWS, 5, 1):
            pieces = stage_rows_padded(nr, seg, lseg, rb, NTH)
            seen = set()
            for lds, glob, r, col in pieces:
                assert 0 <= lds and lds + 16 <= buf
                assert lds == r * lseg + col * 16          # row r at r * lseg
                assert goff + glob + 16 <= nr * rb         # inside the nr rows of the matrix
                assert (r, col) not in seen
                seen.add((r, col))
            assert len(seen) == nr * (seg // 16)
            # furthest read: last byte of the last row's chunk + 4
            assert (nr - 1) * lseg + seg + 4 <= buf


PF_CHUNK, PF_TILE, PF_THREADS = 8, 16, 256
PF_XROW, PF_XROW_AL = PF_CHUNK * 36, PF_CHUNK * 36 + 16


def pf_lds_row(t):
    return {"iq3s": 128, "q6k": 224}.get(t, chunk_bytes(t, PF_CHUNK))


def pf_lds_row_al(t):
    r = pf_lds_row(t)
    return r + 16 if r % 128 == 0 else r


@pytest.mark.parametrize("t,NR,n0", [("q4_0", 128, 64), ("q8_0", 128, 64), ("iq3s", 128, 64), ("iq3s", 128, 128),
                                     ("q4_0", 128, 128), ("q6k", 128, 64), ("q6k", 128, 128)])
def test_prefill_two_stage_padded_slots(t, NR, n0):
    CBL, CBLP = pf_lds_row(t), pf_lds_row_al(t)
    PCB, PCBP, PER, PERP = CBL // 16, CBLP // 16, PF_XROW // 16, PF_XROW_AL // 16
    TW = NR * PCBP
    TWP = (TW + 63) & ~63
    TOT = TWP + PF_TILE * PERP
    wbuf = NR * CBLP + 16          # pf_wst
    xbuf = PF_TILE * PF_XROW_AL    # PF_XST
    NIT = (TOT + PF_THREADS - 1) // PF_THREADS
    wseen, xseen = set(), set()
    for tid in range(PF_THREADS):
        lane, wave = tid & 63, tid >> 6
        for k in range(NIT):
            c0 = wave * 64 + k * PF_THREADS
            cc = c0 + lane
            if c0 < TWP:
                if cc < TW:
                    row, col = divmod(cc, PCBP)
                    if col < PCB:
                        dst = c0 * 16 + lane * 16
                        assert dst == row * CBLP + col * 16 and dst + 16 <= wbuf
                        assert (row, col) not in wseen
                        wseen.add((row, col))
            elif c0 < TOT:
                xc = cc - TWP
                if xc < PF_TILE * PERP:
                    r, col = divmod(xc, PERP)
                    if col < PER:
                        dst = (c0 - TWP) * 16 + lane * 16
                        assert dst == r * PF_XROW_AL + col * 16 and dst + 16 <= xbuf
                        assert (r, col) not in xseen
                        xseen.add((r, col))
    assert len(wseen) == NR * PCB and len(xseen) == PF_TILE * PER
    # readers: the last row's chunk (at most 14 bytes into its span for IQ3_S
    # and Q6_K) plus a 4-byte unaligned read; the activation metadata / fragments
    span_off = max(c * chunk_bytes(t, PF_CHUNK) % 16 for c in range(16))   # 110- / 210-byte chunks: 14
    assert span_off + chunk_bytes(t, PF_CHUNK) <= CBL   # the chunk fits its span
    assert (NR - 1) * CBLP + span_off + chunk_bytes(t, PF_CHUNK) + 4 <= wbuf
    assert (PF_TILE - 1) * PF_XROW_AL + (PF_CHUNK - 1) * 36 + 36 <= xbuf


@pytest.mark.parametrize("pre", [0, 2, 4, 6, 8, 10, 12, 14])
def test_spans_in_288_byte_slots(pre):
    """stage_spans (common.h) with 18 LDS slots per row, as the double-buffered
    tile stages 16-block IQ3_S chunks (two 110-byte superblocks, starting
    `pre` bytes into a 16-byte granule): 64 rows fit the 18,448-byte buffer,
    every piece of every row once, reads of a row's chunk inside its slot."""
    seg, nrows, minper, TB = 220, 64, 18, 64 * 16 * 18 + 16
    per0 = (pre + seg + 15) >> 4
    per = max(per0, minper)
    assert nrows * per * 16 <= TB
    seen = set()
    for c in range(per * nrows):
        r, col = divmod(c, per)
        if col < per0:
            assert c * 16 == r * per * 16 + col * 16
            seen.add((r, col))
    assert len(seen) == nrows * per0
    # the chunk's last byte (plus a 4-byte unaligned read) stays in the row's slot
    assert pre + seg + 4 <= per * 16


def test_iq3s_sign_folded_codebook_lookup():
    """The one-token expert kernel's IQ3_S lookups in the sign-folded codebook
    (chimere_amd/csrc/common.h: Iq3sSignedGrid, iq3s_levels<true>): entry
    16 i + n is entry i with byte k negated where bit k of n is set, and the
    byte offsets (pr << 6) | ((s * 0x4004) & 0x3C003C) of a perm-packed index
    pair give entries 16 idx + nibble in both 16-bit halves.  Checked against
    the codebook with the signs applied per byte (the decode every other kernel
    and the oracle use), for every entry and sign nibble, and on random blocks."""
    import numpy as np
    import npref
    G = npref.GRID.astype(np.int64)
    tab = np.zeros(8192, np.int64)
    for n in range(16):
        v = np.zeros(512, np.int64)
        for k in range(4):
            b = (G >> (8 * k)) & 255
            v |= (np.where((n >> k) & 1, (256 - b) & 255, b)) << (8 * k)
        tab[np.arange(512) * 16 + n] = v
    for n in range(16):   # every entry, every sign nibble: signed levels
        for k in range(4):
            lv = (G >> (8 * k)) & 255
            got = ((tab[np.arange(512) * 16 + n] >> (8 * k)) & 255).astype(np.int8).astype(np.int64)
            assert (got == np.where((n >> k) & 1, -lv, lv)).all()

    def perm(src0, src1, sel):   # v_perm_b32 with selectors 0..7 (bytes of src1, then src0)
        b = [(src1 >> (8 * i)) & 255 for i in range(4)] + [(src0 >> (8 * i)) & 255 for i in range(4)]
        return sum(b[(sel >> (8 * i)) & 255] << (8 * i) for i in range(4))

    def nib_bits(n):
        return (n * 0x00204081) & 0x01010101

    rng = np.random.default_rng(5)
    for _ in range(2000):
        qs = [int(x) for x in rng.integers(0, 256, 8)]
        qh, sg = int(rng.integers(0, 256)), int(rng.integers(0, 1 << 32))
        qs0 = qs[0] | qs[1] << 8 | qs[2] << 16 | qs[3] << 24
        qs1 = qs[4] | qs[5] << 8 | qs[6] << 16 | qs[7] << 24
        h0, h1 = nib_bits(qh & 15), nib_bits((qh >> 4) & 15)
        for p in range(4):
            pr = perm(h0 if p < 2 else h1, qs0 if p < 2 else qs1, 0x07030602 if p & 1 else 0x05010400)
            t = (((sg >> (8 * p)) & 255) * 0x4004) & 0x003C003C
            ab = ((pr << 6) | t) & 0xFFFFFFFF
            for half, word in ((ab & 0xFFFF, 2 * p), (ab >> 16, 2 * p + 1)):
                assert half % 4 == 0 and half < 32768
                idx = qs[word] | ((qh >> word) & 1) << 8          # entry of word `word`
                nib = (sg >> (4 * word)) & 15                     # its sign nibble
                assert half // 4 == 16 * idx + nib
                want = 0
                for k in range(4):
                    lv = (int(G[idx]) >> (8 * k)) & 255
                    want |= (((256 - lv) & 255) if (nib >> k) & 1 else lv) << (8 * k)
                assert int(tab[half // 4]) == want
