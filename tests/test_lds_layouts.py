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
BYTES = {"q4_0": 18, "q8_0": 34, "iq3s": 110}
ELEMS = {"q4_0": 32, "q8_0": 32, "iq3s": 256}


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
    return 128 if t == "iq3s" else chunk_bytes(t, PF_CHUNK)


def pf_lds_row_al(t):
    r = pf_lds_row(t)
    return r + 16 if r % 128 == 0 else r


@pytest.mark.parametrize("t,NR,n0", [("q4_0", 128, 64), ("q8_0", 128, 64), ("iq3s", 128, 64), ("iq3s", 128, 128),
                                     ("q4_0", 128, 128)])
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
    # readers: the last row's chunk (at most 14 bytes into its span for IQ3_S)
    # plus a 4-byte unaligned read; the activation metadata / fragments
    span_off = 14 if t == "iq3s" else 0   # (c * CB) % 16: nonzero only for 110-byte chunks
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
