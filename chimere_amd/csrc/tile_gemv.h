// tile_gemv.h -- the LDS-staged GEMV tile shared by the standalone GEMV and
// the MoE kernels.
//
// A tile is RG*RPG rows handled by RG row groups of 16 lanes (RG*16 threads);
// group g computes rows g, g+RG, ... (RPG of them).  A row is consumed in
// chunks of ChunkGeom<T>::BLOCKS 32-element blocks (a multiple of 16): the
// tile's row segments of a chunk are streamed HBM -> LDS with the widest
// aligned loads, the chunk's Q8_1 activation blocks are decoded once into LDS,
// then lane j of a group takes blocks j, j+16, j+32, ... of the chunk.
// fp32 order (L=16, G=1): per lane acc = fmaf(f32(d_w)*f32(d_x), (float)sumi,
// acc) over its blocks in ascending order, then the 16 lanes are summed with
// the halving tree xor 8,4,2,1 (slot_reduce16).  sumi is the exact int32
// block dot.  Q4_K / Q5_K blocks add a second fmaf for their min term (wacc).
#pragma once
#include <type_traits>
#include "common.h"

namespace chimere {

// Bytes of `blocks` 32-element blocks of a type-T row (256-element
// superblock types: whole superblocks, blocks a multiple of 8).
template <int T>
__host__ __device__ constexpr int chunk_bytes(int blocks) {
    return QTraits<T>::ELEMS == 256 ? blocks / 8 * QTraits<T>::BYTES : blocks * QTraits<T>::BYTES;
}
// Row chunks whose pieces may be only 4-byte aligned (superblocks of 110 or
// 210 bytes, 17-byte blocks): staged with the dword asynchronous copy.
template <int T>
constexpr bool stage_dw() { return T == T_IQ3_S || T == T_Q6_K || T == T_MXFP4; }

template <int T>
struct ChunkGeom {
    // Q8_0 rows are 34 B per block: 32 blocks per chunk keeps 64-row tiles in LDS
    static constexpr int BLOCKS = T == T_Q8_0 ? 32 : 64;
    static constexpr int BYTES = chunk_bytes<T>(BLOCKS);
};
constexpr int MAX_CHUNK_BLOCKS = 64;

// Decoded Q8_1 blocks in LDS
struct XLds {
    int q[8];
    float d;
    int sumq;
};

__device__ __forceinline__ void xlds_to_blk(const XLds& s, XBlk& x) {
#pragma unroll
    for (int k = 0; k < 8; k++) x.q[k] = s.q[k];
    x.d = s.d;
    x.sumq = s.sumq;
}

// The dots of one staged chunk: rows [0, nr) of the tile (LDS row stride
// lseg) against the chunk's cb decoded activation blocks per token.  KC > 0:
// a full chunk of a compile-time row stride KC and CBLK blocks (the block loop
// kept rolled: unrolled it holds more registers and measured slower);
// CHECK: some of the tile's rows are absent (nr < RG*RPG).
template <int T, int NT, int RG, int RPG, int CBLK, int KC, bool CHECK>
__device__ __forceinline__ void tile_compute(const uint8_t* __restrict__ tl, int lseg_rt, int cb_rt,
                                             const XLds* __restrict__ xs, const uint32_t* __restrict__ grid,
                                             int nr, int ntok, float (&acc)[RPG][NT]) {
    const int tid = threadIdx.x;
    const int g = tid >> 4, j = tid & 15;
    const int lseg = KC ? KC : lseg_rt, cb = KC ? CBLK : cb_rt;
    if constexpr (NT == 1) {
        // one token: the activation block is read once for all RPG rows
#pragma unroll 1
        for (int b = j; b < cb; b += SLOTS) {
            XBlk xb;
            xlds_to_blk(xs[b], xb);
#pragma unroll
            for (int r = 0; r < RPG; r++) {
                const int row_i = g + RG * r;
                if (!CHECK || row_i < nr) {
                    WBlk wb;
                    block_decode<T>(tl + row_i * lseg, b, grid, wb);
                    acc[r][0] = wacc<T>(wb, xb, acc[r][0]);
                }
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < RPG; r++) {
            const int row_i = g + RG * r;
            if (!CHECK || row_i < nr) {
                const uint8_t* row = tl + row_i * lseg;
#pragma unroll 1
                for (int b = j; b < cb; b += SLOTS) {
                    WBlk wb;   // decoded once, used for every token
                    block_decode<T>(row, b, grid, wb);
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        if (t < ntok) {
                            XBlk xb;
                            xlds_to_blk(xs[t * CBLK + b], xb);
                            acc[r][t] = wacc<T>(wb, xb, acc[r][t]);
                        }
                    }
                }
            }
        }
    }
}

// One K chunk of tile_gemv (below): blocks [b0, b0 + cb) of the tile's rows.
// FAST: a full chunk (cb == CBLK) with 16-byte aligned pieces, staged by
// stage_rows_fixed (the copies issued back to back) and computed with a
// compile-time row stride and block count; otherwise the general path.
template <int T, int NT, int RG, int RPG, int CBLK, int CPOL, int PAD, bool FAST>
__device__ __forceinline__ void tile_chunk(uint8_t* __restrict__ tile, XLds* __restrict__ xs,
                                           const uint32_t* __restrict__ grid, const uint8_t* base1, int n1,
                                           const uint8_t* base2, int n2, int64_t rb, int b0, int cb,
                                           const uint8_t* __restrict__ X, int64_t x_tok_stride, const int* toks,
                                           int ntok, float (&acc)[RPG][NT]) {
    constexpr int NTH = RG * SLOTS;
    constexpr int CB = chunk_bytes<T>(CBLK);
    const int tid = threadIdx.x;
    const int nr = n1 + n2;
    const int seg = chunk_bytes<T>(cb);
    const int64_t goff = (int64_t)b0 / (QTraits<T>::ELEMS / QK) * QTraits<T>::BYTES;
    // LDS row stride: seg (== CB except in a ragged last chunk), + PAD for
    // 16-byte pieces from 16-byte aligned rows (always so on the FAST path)
    const int lseg = PAD && (FAST || (((seg | goff) & 15) == 0 &&
                                      (((uintptr_t)base1 | (uintptr_t)rb | (uintptr_t)tile) & 15) == 0 &&
                                      (n2 == 0 || ((uintptr_t)base2 & 15) == 0)))
                         ? seg + PAD
                         : seg;
    __syncthreads();   // previous users of tile / xs are done
    if constexpr (FAST) {
        static_assert(CB % 16 == 0, "16-byte pieces");
        if (n2 == 0)
            stage_rows_fixed<CB, CB + PAD, 16, RG * RPG, NTH, CPOL, true>(tile, base1 + goff, n1, nullptr, rb, nr, tid);
        else
            stage_rows_fixed<CB, CB + PAD, 16, RG * RPG, NTH, CPOL>(tile, base1 + goff, n1, base2 + goff, rb, nr, tid);
    } else {
        if (n1) stage_rows<stage_dw<T>(), CPOL>(tile, base1 + goff, rb, n1, seg, tid, NTH, lseg);
        if (n2) stage_rows<stage_dw<T>(), CPOL>(tile + n1 * lseg, base2 + goff, rb, n2, seg, tid, NTH, lseg);
    }
    for (int i = tid; i < ntok * cb; i += NTH) {
        const int t = i / cb, b = i - t * cb;
        const int tk = toks ? toks[t] : t;
        XBlk xb;
        load_xblk(X + tk * x_tok_stride + (int64_t)(b0 + b) * Q8_1_BYTES, xb);
        XLds& o = xs[t * CBLK + b];
#pragma unroll
        for (int k = 0; k < 8; k++) o.q[k] = xb.q[k];
        o.d = xb.d;
        o.sumq = T == T_Q4_0S ? (int)xb.sbits : xb.sumq;   // the s-form needs s, not the quant sum
    }
    lds_copy_wait();
    __syncthreads();
    if constexpr (FAST) {
        if (nr == RG * RPG)
            tile_compute<T, NT, RG, RPG, CBLK, CB + PAD, false>(tile, 0, 0, xs, grid, nr, ntok, acc);
        else
            tile_compute<T, NT, RG, RPG, CBLK, CB + PAD, true>(tile, 0, 0, xs, grid, nr, ntok, acc);
    } else {
        tile_compute<T, NT, RG, RPG, CBLK, 0, true>(tile, lseg, cb, xs, grid, nr, ntok, acc);
    }
}

// Accumulates per-lane partial dots for the rows of a tile against up to NT
// tokens.  Tile rows [0, n1) come from base1, rows [n1, n1+n2) from base2
// (global row stride rb for both); n1 + n2 <= RG*RPG.  Token i's Q8_1 row is
// at X + tok(i) * x_tok_stride with tok(i) = toks ? toks[i] : i.
// acc[r][t]: partial sum of the group's r-th row (tile row g + RG*r) for
// token t; reduce with slot_reduce16.  Contains __syncthreads().
// CBLK: blocks per chunk (default ChunkGeom<T>::BLOCKS; a multiple of 16,
// and of 8 for IQ3_S); xs holds NT * CBLK decoded blocks (token-major).
// CPOL: cache policy of the weight copies (2 = non-temporal: weights are
// streamed once per call).
// PAD: bytes added to the LDS row stride of 16-byte multiple chunk rows, so
// that the rows a wave reads at once start on different banks (the tile
// buffer then needs rows * (chunk bytes + PAD))
// FIX: full 16-byte aligned chunks on tile_chunk's FAST path (measured
// faster for the standalone GEMV, slower -- more registers -- in the MoE
// kernels' tiles)
template <int T, int NT, int RG, int RPG, int CBLK = ChunkGeom<T>::BLOCKS, int CPOL = 0, int PAD = 0,
          bool FIX = false>
__device__ __forceinline__ void tile_gemv(uint8_t* __restrict__ tile, XLds* __restrict__ xs,
                                          const uint32_t* __restrict__ grid,
                                          const uint8_t* base1, int n1, const uint8_t* base2, int n2,
                                          int64_t rb, int ncols, const uint8_t* __restrict__ X,
                                          int64_t x_tok_stride, const int* toks, int ntok,
                                          float (&acc)[RPG][NT]) {
    static_assert(CBLK % SLOTS == 0 && (QTraits<T>::ELEMS != 256 || CBLK % 8 == 0) && CBLK <= MAX_CHUNK_BLOCKS, "chunk");
    const int nb = ncols / QK;
#pragma unroll
    for (int r = 0; r < RPG; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
    constexpr bool FIXOK = FIX && chunk_bytes<T>(CBLK) % 16 == 0;
    const bool al16 = (((uintptr_t)base1 | (uintptr_t)rb | (uintptr_t)tile) & 15) == 0 &&
                      (n2 == 0 || ((uintptr_t)base2 & 15) == 0);
    for (int b0 = 0; b0 < nb; b0 += CBLK) {
        // chunk offsets are multiples of the (16-byte multiple) chunk bytes
        if (FIXOK && al16 && nb - b0 >= CBLK)
            tile_chunk<T, NT, RG, RPG, CBLK, CPOL, PAD, FIXOK>(tile, xs, grid, base1, n1, base2, n2, rb, b0, CBLK, X,
                                                               x_tok_stride, toks, ntok, acc);
        else
            tile_chunk<T, NT, RG, RPG, CBLK, CPOL, PAD, false>(tile, xs, grid, base1, n1, base2, n2, rb, b0,
                                                               min(CBLK, nb - b0), X, x_tok_stride, toks, ntok,
                                                               acc);
    }
}

}  // namespace chimere

namespace chimere {

// Q8_1 block from raw bytes in LDS (36 bytes, 4-byte aligned); the sum of the
// quants only where the weight type needs it (Q4_0, Q4_K, Q5_K).
template <int T>
__device__ __forceinline__ void raw_xblk(const uint8_t* p, XBlk& x) {
    const uint32_t* w = (const uint32_t*)p;
    x.d = h2f(w[0] & 0xFFFFu);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        x.q[i] = (int)w[1 + i];
        if constexpr (needs_sumq<T>()) s = dot4(x.q[i], 0x01010101, s);
    }
    x.sumq = s;
}

// tile_gemv with double-buffered K chunks: chunk c+1 (weight rows and the
// tokens' raw Q8_1 blocks, both by asynchronous global->LDS copies) is in
// flight while chunk c is computed.  tile: 2 buffers of TB bytes (TB >=
// (n1+n2) * chunk_bytes<T>(CBLK)); xraw: 2 buffers of NT * CBLK * 36 bytes.
// Needs 16-byte aligned row starts and chunk offsets (rb, X, x_tok_stride
// multiples of 16; ncols a multiple of 128).  Same fp32 order as tile_gemv.
template <int T, int NT, int RG, int RPG, int CBLK, int CPOL = 0>
__device__ __forceinline__ void tile_gemv_db(uint8_t* __restrict__ tile, int TB, uint8_t* __restrict__ xraw,
                                             const uint32_t* __restrict__ grid, const uint8_t* base1, int n1,
                                             const uint8_t* base2, int n2, int64_t rb, int ncols,
                                             const uint8_t* __restrict__ X, int64_t x_tok_stride, const int* toks,
                                             int ntok, float (&acc)[RPG][NT]) {
    constexpr int NTH = RG * SLOTS, XB = NT * CBLK * Q8_1_BYTES;
    static_assert(CBLK % SLOTS == 0 && (QTraits<T>::ELEMS != 256 || CBLK % 8 == 0) && CBLK <= MAX_CHUNK_BLOCKS, "chunk");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = tid >> 4, j = tid & 15;
    const int nr = n1 + n2;
    const int nb = ncols / QK, nc = (nb + CBLK - 1) / CBLK;
#pragma unroll
    for (int r = 0; r < RPG; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
    // 16-byte aligned spans of 4-byte aligned rows (IQ3_S, Q6_K, MXFP4 chunks)
    // where they fit the buffer: 16-byte copies instead of dword ones
    // IQ3_S chunks of 16 blocks: LDS rows of up to 288 bytes (the spans need
    // 224 or 240), the most the buffer holds (the several-token gate/up's
    // buffers hold 240-byte rows: its M=8 layer 48.4 -> 48.0 us against 272)
    constexpr int SPER0 = T == T_IQ3_S && CBLK == 16 ? 18 : 0;
    const int SPER = SPER0 && nr * 16 * SPER0 > TB ? (TB - 16) / (nr * 16) : SPER0;
    const bool spans = stage_dw<T>() && (rb & 15) == 0 && (n2 == 0 || (((uintptr_t)base1 ^ (uintptr_t)base2) & 15) == 0) &&
                       nr * max((chunk_bytes<T>(CBLK) + 30) / 16 * 16, 16 * SPER) <= TB;
    int pre0 = 0, pre1 = 0, rs0 = 0, rs1 = 0;   // per buffer: data offset and LDS row stride
    auto issue = [&](int c, int buf) {
        const int b0 = c * CBLK, cb = min(CBLK, nb - b0);
        const int seg = chunk_bytes<T>(cb);
        const int64_t goff = (int64_t)b0 / (QTraits<T>::ELEMS / QK) * QTraits<T>::BYTES;
        uint8_t* tb = tile + buf * TB;
        // token t's cb blocks at xraw + buf*XB + t*cb*36 (16-byte pieces)
        const int per = cb * Q8_1_BYTES / 16, tot = ntok * per;
        uint8_t* xb = xraw + buf * XB;
        auto xsrc = [&](int cc) {
            const int t = cc / per, col = cc - t * per;
            const int tk = toks ? toks[t] : t;
            return X + tk * x_tok_stride + (int64_t)b0 * Q8_1_BYTES + col * 16;
        };
        if (spans) {
            int rs;
            const int pre = stage_spans<CPOL>(tb, base1 + goff, n1, base2 + goff, n2, rb, seg, &rs, xb, tot, xsrc,
                                              tid, NTH, SPER);
            if (buf) { pre1 = pre; rs1 = rs; } else { pre0 = pre; rs0 = rs; }
            return;
        }
        if (buf) { pre1 = 0; rs1 = seg; } else { pre0 = 0; rs0 = seg; }
        if (n1) stage_rows<stage_dw<T>(), CPOL>(tb, base1 + goff, rb, n1, seg, tid, NTH);
        if (n2) stage_rows<stage_dw<T>(), CPOL>(tb + n1 * seg, base2 + goff, rb, n2, seg, tid, NTH);
        for (int c0 = wave * 64; c0 < tot; c0 += NTH) {
            const int cc = c0 + lane;
            if (cc < tot) {
                const int t = cc / per, col = cc - t * per;
                const int tk = toks ? toks[t] : t;
                __builtin_amdgcn_global_load_lds(
                    (const glb_void_t*)(X + tk * x_tok_stride + (int64_t)b0 * Q8_1_BYTES + col * 16),
                    (lds_void_t*)(xb + c0 * 16), 16, 0, 0);
            }
        }
    };
    issue(0, 0);
    for (int c = 0; c < nc; c++) {
        const int buf = c & 1, cb = min(CBLK, nb - c * CBLK);
        lds_copy_wait();
        __syncthreads();   // chunk c landed; every wave is done with chunk c-1
        if (c + 1 < nc) issue(c + 1, buf ^ 1);
        const uint8_t* tb = tile + buf * TB + (buf ? pre1 : pre0);
        const int seg = buf ? rs1 : rs0;   // LDS row stride of this chunk
        const uint8_t* xb = xraw + buf * XB;
        // the chunk's activation blocks of the (at most NT) tokens are read
        // once for all RPG rows; each (row, token) still accumulates its
        // blocks in ascending order
        // a full tile (every row group holds RPG rows, NT tokens) runs
        // without the per-row and per-token guards, so the rows' block
        // decodes are straight-line code the compiler can interleave (one
        // row's LDS reads under another's arithmetic)
        auto blocks = [&](auto full) {
            for (int b = j; b < cb; b += SLOTS) {
                XBlk x[NT];
#pragma unroll
                for (int t = 0; t < NT; t++)
                    if (decltype(full)::value || t < ntok) raw_xblk<T>(xb + (t * cb + b) * Q8_1_BYTES, x[t]);
#pragma unroll
                for (int r = 0; r < RPG; r++) {
                    const int row_i = g + RG * r;
                    if (decltype(full)::value || row_i < nr) {
                        WBlk wb;
                        block_decode<T>(tb + __mul24(row_i, seg), b, grid, wb);
#pragma unroll
                        for (int t = 0; t < NT; t++)
                            if (decltype(full)::value || t < ntok) acc[r][t] = wacc<T>(wb, x[t], acc[r][t]);
                    }
                }
            }
        };
        // full: every row group holds RPG rows and the item has NT tokens
        if (nr == RG * RPG && ntok == NT) blocks(std::true_type{});
        else blocks(std::false_type{});
    }
}

}  // namespace chimere
