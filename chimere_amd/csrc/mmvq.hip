// mmvq.hip -- block-quantized GEMV (Q8_0 / Q4_0 / IQ3_S / Q4_K / Q5_K / Q6_K /
// MXFP4 weights x Q8_1 activations) for 1..8 tokens, plain /
// batched-by-expert-id / debug dots.
//
// Work-group = 256 threads = 16 row groups of 16 lanes; one tile = 16
// consecutive rows, streamed through LDS by tile_gemv (which documents the
// fp32 order: L=16 lanes per row, G=1).
#include "api_internal.h"
#include "common.h"
#include "tile_gemv.h"

namespace chimere {

void launch_quantize_q8_1(const float* x, void* out, int64_t ncols, int64_t ncols_padded,
                          int64_t nrows, hipStream_t s);

extern __constant__ uint32_t c_iq3s_grid_mmvq[512];
__constant__ uint32_t c_iq3s_grid_mmvq[512] = CHIMERE_IQ3S_GRID_INIT;

struct MmvqArgs {
    const uint8_t* W;
    const uint8_t* x;
    float* y;
    int ncols, nrows, ntok;
    int64_t x_tok_stride;   // bytes between tokens' Q8_1 rows
    int64_t y_tok_stride;   // floats between tokens' outputs
    const int* ids;         // slot k -> expert ids[k]; NULL: expert k
    int64_t w_slot_stride;  // bytes per expert
    int64_t x_slot_stride;  // bytes between slots' inputs (0: shared)
    int64_t y_slot_stride;  // floats between slots' outputs
};

// Blocks per K chunk of the GEMV tile: 64 for every type, which puts a
// 2048-column Q8_0 row in one chunk (one exposed round trip per work-group
// instead of two: 4096 x 2048 5.45 -> 4.75 us).  Larger chunks for the
// K-quants / MXFP4 (a 4096-column row in one) and the double-buffered tile
// with 32- or 64-block chunks were measured slower: fewer work-groups fit a
// CU, and at 64 blocks four are resident per CU already.
constexpr int MMVQ_BLOCKS = 64;

// LDS row padding of the tile (bytes): with it the 4 rows a wave reads at
// once start on different banks (from a model of the block reads' bank
// conflicts: Q4_0 1152 -> 1200 B, Q8_0 2176 -> 2224 B, IQ3_S 880 -> 960 B)
template <int T>
constexpr int mmvq_pad() { return T == T_Q4_0 || T == T_Q4_0S || T == T_Q8_0 ? 48 : (T == T_IQ3_S ? 80 : 0); }

template <int T, int NTOK>
__global__ __launch_bounds__(GEMV_THREADS) void k_mmvq(MmvqArgs a) {
    constexpr int CBLK = MMVQ_BLOCKS;
    constexpr int CB = chunk_bytes<T>(CBLK), PAD = mmvq_pad<T>();
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE_ROWS * (CB + PAD) + 16];
    __shared__ XLds xs[NTOK][CBLK];
    __shared__ uint32_t grid[T == T_IQ3_S ? 512 : 1];

    const int tid = threadIdx.x;
    const int g = tid >> 4, j = tid & 15;
    const int slot = blockIdx.y;
    const int r0 = blockIdx.x * TILE_ROWS;
    const int nr = min(TILE_ROWS, a.nrows - r0);
    const int64_t e = a.ids ? (int64_t)a.ids[slot] : (int64_t)slot;
    const int64_t rb = row_bytes(T == T_Q4_0S ? T_Q4_0 : T, a.ncols);
    if constexpr (T == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_mmvq[i];

    float acc[1][NTOK];
    tile_gemv<T, NTOK, TILE_ROWS, 1, CBLK, CPOL_STREAM, PAD, true>(tile, &xs[0][0], grid,
                                     a.W + e * a.w_slot_stride + (int64_t)r0 * rb, nr,
                                     nullptr, 0, rb, a.ncols, a.x + slot * a.x_slot_stride, a.x_tok_stride,
                                     nullptr, a.ntok, acc);
    if (g < nr) {
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            if (t < a.ntok) {
                const float v = slot_reduce16(acc[0][t]);
                if (j == 0) a.y[slot * a.y_slot_stride + t * a.y_tok_stride + r0 + g] = v;
            }
        }
    }
}

// One token, rows of exactly NCH 64-block chunks (2048 * NCH columns), whole
// 16-row tiles, 16-byte aligned rows: the tile's copies, the activation
// blocks, the dots and the L=16 tree with compile-time sizes and a
// compile-time chunk count (the same fp32 order as tile_gemv; the general
// path's run-time row count and chunk loop cost ~0.35 us of latency per
// launch: Q8_0 4096x2048 4.24 -> 3.90 us, Q4_0 head 30.8 -> 28.6 us).
template <int T, int NCH>
__global__ __launch_bounds__(GEMV_THREADS) void k_mmvq_nc(MmvqArgs a) {
    constexpr int CBLK = MMVQ_BLOCKS, CB = chunk_bytes<T>(CBLK), LS = CB + mmvq_pad<T>();
    static_assert(CB % 16 == 0, "16-byte pieces");
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE_ROWS * LS + 16];
    __shared__ XLds xs[CBLK];
    __shared__ uint32_t grid[T == T_IQ3_S ? 512 : 1];
    const int tid = threadIdx.x, g = tid >> 4, j = tid & 15;
    const int slot = blockIdx.y;
    const int64_t e = a.ids ? (int64_t)a.ids[slot] : (int64_t)slot;
    constexpr int64_t RB = (int64_t)NCH * CB;
    const uint8_t* W = a.W + e * a.w_slot_stride + (int64_t)blockIdx.x * TILE_ROWS * RB;
    const uint8_t* X = a.x + slot * a.x_slot_stride;
    if constexpr (T == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_mmvq[i];
    float acc = 0.0f;
#pragma unroll 1
    for (int c = 0; c < NCH; c++) {
        if (c > 0) __syncthreads();   // every wave is done with the previous chunk
        stage_rows_fixed<CB, LS, 16, TILE_ROWS, GEMV_THREADS, CPOL_STREAM, true>(tile, W + c * CB, TILE_ROWS, nullptr,
                                                                                  RB, TILE_ROWS, tid);
        if (tid < CBLK) {
            XBlk xb;
            load_xblk(X + (int64_t)(c * CBLK + tid) * Q8_1_BYTES, xb);
            XLds& o = xs[tid];
#pragma unroll
            for (int k = 0; k < 8; k++) o.q[k] = xb.q[k];
            o.d = xb.d;
            o.sumq = T == T_Q4_0S ? (int)xb.sbits : xb.sumq;
        }
        lds_copy_wait();
        __syncthreads();
#pragma unroll 1
        for (int b = j; b < CBLK; b += SLOTS) {
            XBlk xb;
            xlds_to_blk(xs[b], xb);
            WBlk wb;
            block_decode<T>(tile + g * LS, b, grid, wb);
            acc = wacc<T>(wb, xb, acc);
        }
    }
    const float v = slot_reduce16(acc);
    if (j == 0) a.y[slot * a.y_slot_stride + blockIdx.x * TILE_ROWS + g] = v;
}

template <int T>
static void launch_t(const MmvqArgs& a, int nslots, hipStream_t s) {
    dim3 grid((unsigned)((a.nrows + TILE_ROWS - 1) / TILE_ROWS), (unsigned)nslots);
    if constexpr (chunk_bytes<T>(MMVQ_BLOCKS) % 16 == 0) {
        const int nch = a.ncols / (MMVQ_BLOCKS * QK);
        if (a.ntok == 1 && a.ncols % (MMVQ_BLOCKS * QK) == 0 && (nch == 1 || nch == 2) && a.nrows % TILE_ROWS == 0 &&
            (((uintptr_t)a.W | (uintptr_t)a.w_slot_stride) & 15) == 0) {
            if (nch == 1) hipLaunchKernelGGL((k_mmvq_nc<T, 1>), grid, dim3(GEMV_THREADS), 0, s, a);
            else hipLaunchKernelGGL((k_mmvq_nc<T, 2>), grid, dim3(GEMV_THREADS), 0, s, a);
            return;
        }
    }
    dim3 blk(GEMV_THREADS);
    switch (a.ntok) {
#define CASE(N) case N: hipLaunchKernelGGL((k_mmvq<T, N>), grid, blk, 0, s, a); break;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
#undef CASE
    }
}

bool launch_mmvq(int type, const MmvqArgs& a, int nslots, hipStream_t s) {
    switch (type) {
    case T_Q8_0: launch_t<T_Q8_0>(a, nslots, s); break;
    case T_Q4_0: launch_t<T_Q4_0>(a, nslots, s); break;
    case T_Q4_0S: launch_t<T_Q4_0S>(a, nslots, s); break;
    case T_IQ3_S: launch_t<T_IQ3_S>(a, nslots, s); break;
    case T_Q4_K: launch_t<T_Q4_K>(a, nslots, s); break;
    case T_Q5_K: launch_t<T_Q5_K>(a, nslots, s); break;
    case T_Q6_K: launch_t<T_Q6_K>(a, nslots, s); break;
    case T_MXFP4: launch_t<T_MXFP4>(a, nslots, s); break;
    default: return false;
    }
    return true;
}

// Validates a GEMV request; returns false (error recorded) when rejected.
static bool check_gemv(const char* who, int type, const void* W, const void* x, const float* y,
                       int ncols, int nrows, int nrows_y_padded, int ntok) {
    if (!W || !x || !y) { set_error(CHIMERE_ERR_ARG, "%s: null pointer", who); return false; }
    if (type_block_bytes(type) == 0) {
        set_error(CHIMERE_ERR_ARG, "%s: unsupported type %d", who, type); return false;
    }
    const int elems = type_block_elems(type);
    if (ncols <= 0 || nrows <= 0 || ncols % elems) {
        set_error(CHIMERE_ERR_ARG, "%s: ncols=%d must be a positive multiple of %d (nrows=%d)",
                  who, ncols, elems, nrows);
        return false;
    }
    if (nrows_y_padded < ncols / 32) {
        set_error(CHIMERE_ERR_ARG, "%s: nrows_y_padded=%d < ncols/32=%d", who, nrows_y_padded, ncols / 32);
        return false;
    }
    if (ntok < 1 || ntok > 8) { set_error(CHIMERE_ERR_ARG, "%s: ntok=%d not in 1..8", who, ntok); return false; }
    // MXFP4's 17-byte blocks have no alignment; every other block starts with an f16
    if (((uintptr_t)x & 3) != 0 || (type != T_MXFP4 && ((uintptr_t)W & 1) != 0)) {
        set_error(CHIMERE_ERR_ARG, "%s: Q8_1 input must be 4-byte and weights 2-byte aligned", who);
        return false;
    }
    return true;
}

static void gemv_entry(const char* who, int type, const void* W, const void* x, float* y, int ncols,
                       int nrows, int nrows_y_padded, int ntok, hipStream_t s) {
    // the s-form GEMV reads plain Q4_0 blocks
    if (!check_gemv(who, type == T_Q4_0S ? T_Q4_0 : type, W, x, y, ncols, nrows, nrows_y_padded, ntok)) return;
    MmvqArgs a{(const uint8_t*)W, (const uint8_t*)x, y, ncols, nrows, ntok,
               (int64_t)nrows_y_padded * Q8_1_BYTES, nrows, nullptr, 0, 0, 0};
    launch_mmvq(type, a, 1, s);
    check_launch(who);
}

static void gemv_f32_entry(const char* who, int type, const void* W, const float* x, float* y,
                           int ncols, int nrows, int ncols_padded, void* scratch, hipStream_t s) {
    if (!x || !scratch) { set_error(CHIMERE_ERR_ARG, "%s: null pointer", who); return; }
    if (ncols_padded < ncols || ncols_padded % 32) {
        set_error(CHIMERE_ERR_ARG, "%s: ncols_padded=%d invalid for ncols=%d", who, ncols_padded, ncols);
        return;
    }
    if (!check_gemv(who, type, W, scratch, y, ncols, nrows, ncols_padded / 32, 1)) return;
    launch_quantize_q8_1(x, scratch, ncols, ncols_padded, 1, s);
    gemv_entry(who, type, W, scratch, y, ncols, nrows, ncols_padded / 32, 1, s);
}

static void gemv_batched_entry(const char* who, int type, const void* W, const void* x, float* y,
                               const int* ids, int ncols, int nrows, int nrows_y_padded,
                               int64_t expert_stride, int64_t input_stride, int top_k,
                               hipStream_t s) {
    if (!check_gemv(who, type, W, x, y, ncols, nrows, nrows_y_padded, 1)) return;
    if (!ids || top_k <= 0 || expert_stride < row_bytes(type, ncols) * nrows || input_stride < 0 ||
        (input_stride & 3)) {
        set_error(CHIMERE_ERR_ARG, "%s: bad ids/top_k/strides (top_k=%d expert_stride=%lld input_stride=%lld)",
                  who, top_k, (long long)expert_stride, (long long)input_stride);
        return;
    }
    MmvqArgs a{(const uint8_t*)W, (const uint8_t*)x, y, ncols, nrows, 1,
               0, 0, ids, expert_stride, input_stride, nrows};
    launch_mmvq(type, a, top_k, s);
    check_launch(who);
}

// ---- debug: exact int32 per-block dots, one thread per (row, block).
// Q4_K / Q5_K: the scaled quant dot sc * sum(q*q_x) (the block's min term is
// m * sum(q_x), a function of the scale bytes and the activation alone).
template <int T>
__global__ void k_block_dots(const uint8_t* __restrict__ W, const uint8_t* __restrict__ x,
                             int32_t* __restrict__ out, int ncols, int nrows) {
    __shared__ uint32_t grid[T == T_IQ3_S ? 512 : 1];
    if constexpr (T == T_IQ3_S)
        for (int i = threadIdx.x; i < 512; i += blockDim.x) grid[i] = c_iq3s_grid_mmvq[i];
    __syncthreads();
    const int nb = ncols / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)nb * nrows) return;
    const int r = (int)(i / nb), b = (int)(i % nb);
    const uint8_t* row = W + (int64_t)r * row_bytes(T, ncols);
    // the block (or its superblock) copied to a private 4-byte aligned buffer
    constexpr int SUPER = QTraits<T>::ELEMS == 256;
    constexpr int LEN = QTraits<T>::BYTES;
    uint8_t buf[(LEN + 7) / 4 * 4] __attribute__((aligned(4)));
    const int64_t off = SUPER ? (int64_t)(b >> 3) * LEN : (int64_t)b * LEN;
    for (int k = 0; k < LEN; k++) buf[k] = row[off + k];
    for (int k = LEN; k < (int)sizeof(buf); k++) buf[k] = 0;
    XBlk xb;
    load_xblk(x + (int64_t)b * Q8_1_BYTES, xb);
    WBlk w;
    block_decode<T>(buf, SUPER ? (b & 7) : 0, grid, w);
    out[i] = wdot<T>(w, xb);
}

template <int T>
static void launch_block_dots(const void* w, const void* x, int32_t* out, int ncols, int nrows, hipStream_t s) {
    const int64_t n = (int64_t)(ncols / 32) * nrows;
    hipLaunchKernelGGL((k_block_dots<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint8_t*)w,
                       (const uint8_t*)x, out, ncols, nrows);
}

}  // namespace chimere

using namespace chimere;

extern "C" {

void chimere_mmvq_iq3s(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_iq3s", T_IQ3_S, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_q8_0(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_q8_0", T_Q8_0, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_q4_0(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_q4_0", T_Q4_0, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_q4_0_sform(const void* w, const void* x, float* y, int ncols, int nrows, int nyp,
                             hipStream_t s) {
    gemv_entry("mmvq_q4_0_sform", T_Q4_0S, w, x, y, ncols, nrows, nyp, 1, s);
}

void chimere_mmvq_iq3s_f32(const void* w, const float* x, float* y, int ncols, int nrows, int ncp,
                           void* scratch, hipStream_t s) {
    gemv_f32_entry("mmvq_iq3s_f32", T_IQ3_S, w, x, y, ncols, nrows, ncp, scratch, s);
}
void chimere_mmvq_q8_0_f32(const void* w, const float* x, float* y, int ncols, int nrows, int ncp,
                           void* scratch, hipStream_t s) {
    gemv_f32_entry("mmvq_q8_0_f32", T_Q8_0, w, x, y, ncols, nrows, ncp, scratch, s);
}
void chimere_mmvq_q4_0_f32(const void* w, const float* x, float* y, int ncols, int nrows, int ncp,
                           void* scratch, hipStream_t s) {
    gemv_f32_entry("mmvq_q4_0_f32", T_Q4_0, w, x, y, ncols, nrows, ncp, scratch, s);
}

void chimere_mmvq_iq3s_batched(const void* w, const void* x, float* y, const int* ids, int ncols,
                               int nrows, int nyp, int64_t es, int64_t is, int top_k, hipStream_t s) {
    gemv_batched_entry("mmvq_iq3s_batched", T_IQ3_S, w, x, y, ids, ncols, nrows, nyp, es, is, top_k, s);
}
void chimere_mmvq_q8_0_batched(const void* w, const void* x, float* y, const int* ids, int ncols,
                               int nrows, int nyp, int64_t es, int64_t is, int top_k, hipStream_t s) {
    gemv_batched_entry("mmvq_q8_0_batched", T_Q8_0, w, x, y, ids, ncols, nrows, nyp, es, is, top_k, s);
}
void chimere_mmvq_q4_0_batched(const void* w, const void* x, float* y, const int* ids, int ncols,
                               int nrows, int nyp, int64_t es, int64_t is, int top_k, hipStream_t s) {
    gemv_batched_entry("mmvq_q4_0_batched", T_Q4_0, w, x, y, ids, ncols, nrows, nyp, es, is, top_k, s);
}

// ggml K-quant / MXFP4 entry points (ffi/ggml_cuda_gemv.cu:118-175, 292-460)
void chimere_mmvq_q5k(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_q5k", T_Q5_K, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_q4k(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_q4k", T_Q4_K, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_q6k(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_q6k", T_Q6_K, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_mxfp4(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, hipStream_t s) {
    gemv_entry("mmvq_mxfp4", T_MXFP4, w, x, y, ncols, nrows, nyp, 1, s);
}
void chimere_mmvq_q5k_f32(const void* w, const float* x, float* y, int ncols, int nrows, int ncp, void* scratch,
                          hipStream_t s) {
    gemv_f32_entry("mmvq_q5k_f32", T_Q5_K, w, x, y, ncols, nrows, ncp, scratch, s);
}
void chimere_mmvq_q4k_f32(const void* w, const float* x, float* y, int ncols, int nrows, int ncp, void* scratch,
                          hipStream_t s) {
    gemv_f32_entry("mmvq_q4k_f32", T_Q4_K, w, x, y, ncols, nrows, ncp, scratch, s);
}
void chimere_mmvq_q6k_f32(const void* w, const float* x, float* y, int ncols, int nrows, int ncp, void* scratch,
                          hipStream_t s) {
    gemv_f32_entry("mmvq_q6k_f32", T_Q6_K, w, x, y, ncols, nrows, ncp, scratch, s);
}
// argument order as the reference's: scratch before the output
void chimere_mmvq_mxfp4_f32(const void* w, const float* x, void* scratch, float* y, int ncols, int nrows, int ncp,
                            hipStream_t s) {
    gemv_f32_entry("mmvq_mxfp4_f32", T_MXFP4, w, x, y, ncols, nrows, ncp, scratch, s);
}
// expert ids are read on the device (the reference dereferences them on the host)
void chimere_mmvq_mxfp4_batched(const void* w, const void* x, float* y, const int* ids, int ncols, int nrows,
                                int nyp, int64_t es, int64_t is, int top_k, hipStream_t s) {
    gemv_batched_entry("mmvq_mxfp4_batched", T_MXFP4, w, x, y, ids, ncols, nrows, nyp, es, is, top_k, s);
}

void chimere_mmvq_multi(int type, const void* w, const void* x, float* y, int ncols, int nrows,
                        int nyp, int ntok, hipStream_t s) {
    gemv_entry("mmvq_multi", type, w, x, y, ncols, nrows, nyp, ntok, s);
}

void chimere_mmvq_q4_0_multi(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, int ntok,
                             hipStream_t s) {
    gemv_entry("mmvq_q4_0_multi", T_Q4_0, w, x, y, ncols, nrows, nyp, ntok, s);
}
void chimere_mmvq_q8_0_multi(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, int ntok,
                             hipStream_t s) {
    gemv_entry("mmvq_q8_0_multi", T_Q8_0, w, x, y, ncols, nrows, nyp, ntok, s);
}
void chimere_mmvq_iq3s_multi(const void* w, const void* x, float* y, int ncols, int nrows, int nyp, int ntok,
                             hipStream_t s) {
    gemv_entry("mmvq_iq3s_multi", T_IQ3_S, w, x, y, ncols, nrows, nyp, ntok, s);
}

void chimere_dbg_block_dots(int type, const void* w, const void* x, int32_t* out, int ncols,
                            int nrows, hipStream_t s) {
    if (!out || !check_gemv("dbg_block_dots", type, w, x, (const float*)out, ncols, nrows, ncols / 32, 1))
        return;
    switch (type) {
    case T_Q8_0: launch_block_dots<T_Q8_0>(w, x, out, ncols, nrows, s); break;
    case T_Q4_0: launch_block_dots<T_Q4_0>(w, x, out, ncols, nrows, s); break;
    case T_IQ3_S: launch_block_dots<T_IQ3_S>(w, x, out, ncols, nrows, s); break;
    case T_Q4_K: launch_block_dots<T_Q4_K>(w, x, out, ncols, nrows, s); break;
    case T_Q5_K: launch_block_dots<T_Q5_K>(w, x, out, ncols, nrows, s); break;
    case T_Q6_K: launch_block_dots<T_Q6_K>(w, x, out, ncols, nrows, s); break;
    case T_MXFP4: launch_block_dots<T_MXFP4>(w, x, out, ncols, nrows, s); break;
    }
    check_launch("dbg_block_dots");
}

}  // extern "C"
