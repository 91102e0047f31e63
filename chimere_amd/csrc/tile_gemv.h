// tile_gemv.h -- the 16-row x 16-lane GEMV tile shared by the standalone
// GEMV and the MoE kernels.  See mmvq.hip for the fp32 order it implements.
#pragma once
#include "common.h"

namespace chimere {

template <int T>
struct ChunkGeom {
    static constexpr int BYTES = T == T_IQ3_S ? CHUNK_BLOCKS / 8 * 110 : CHUNK_BLOCKS * QTraits<T>::BYTES;
};

// Decoded Q8_1 blocks in LDS
struct XLds {
    int q[8];
    float d;
    int sumq;
};

// Accumulates, for the 16 rows of a tile, per-lane partial dots against up to
// NT tokens.  Rows [0, n1) come from base1, rows [n1, n1+n2) from base2 (row
// stride rb in both).  Token i's Q8_1 row is at X + tok(i) * x_tok_stride
// where tok(i) = toks ? toks[i] : i.  acc[t] is the lane's partial sum
// (lane j of row group g covers blocks j, j+16, ... in ascending order);
// reduce with slot_reduce16.  Contains __syncthreads(): call from all threads.
template <int T, int NT>
__device__ __forceinline__ void tile_gemv(uint8_t* __restrict__ tile, int lstride,
                                          XLds (*__restrict__ xs)[CHUNK_BLOCKS],
                                          const uint32_t* __restrict__ grid,
                                          const uint8_t* base1, int n1, const uint8_t* base2, int n2,
                                          int64_t rb, int ncols, const uint8_t* __restrict__ X,
                                          int64_t x_tok_stride, const int* toks, int ntok,
                                          float (&acc)[NT]) {
    const int tid = threadIdx.x;
    const int g = tid >> 4, j = tid & 15;
    const int nr = n1 + n2;
    const int nb = ncols / QK;
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += CHUNK_BLOCKS) {
        const int cb = min(CHUNK_BLOCKS, nb - b0);
        const int seg = T == T_IQ3_S ? cb / 8 * 110 : cb * QTraits<T>::BYTES;
        const int64_t goff = T == T_IQ3_S ? (int64_t)b0 / 8 * 110 : (int64_t)b0 * QTraits<T>::BYTES;
        __syncthreads();   // previous users of tile / xs are done
        if (n1) stage_rows(tile, lstride, base1 + goff, rb, n1, seg, tid, GEMV_THREADS);
        if (n2) stage_rows(tile + n1 * lstride, lstride, base2 + goff, rb, n2, seg, tid, GEMV_THREADS);
        for (int i = tid; i < ntok * cb; i += GEMV_THREADS) {
            const int t = i / cb, b = i - t * cb;
            const int tk = toks ? toks[t] : t;
            XBlk xb;
            load_xblk(X + tk * x_tok_stride + (int64_t)(b0 + b) * Q8_1_BYTES, xb);
#pragma unroll
            for (int k = 0; k < 8; k++) xs[t][b].q[k] = xb.q[k];
            xs[t][b].d = xb.d;
            xs[t][b].sumq = xb.sumq;
        }
        __syncthreads();
        if (g < nr) {
            const uint8_t* row = tile + g * lstride;
            for (int b = j; b < cb; b += SLOTS) {
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if (t < ntok) {
                        XBlk xb;
#pragma unroll
                        for (int k = 0; k < 8; k++) xb.q[k] = xs[t][b].q[k];
                        xb.d = xs[t][b].d;
                        xb.sumq = xs[t][b].sumq;
                        float dw;
                        const int s = block_dot<T>(row, b, xb, grid, &dw);
                        acc[t] = __builtin_fmaf(dw * xb.d, (float)s, acc[t]);
                    }
                }
            }
        }
    }
}

}  // namespace chimere
