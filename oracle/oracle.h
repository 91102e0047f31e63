/*
 * oracle.h -- CPU restatement of the reference's decode-time quantized
 * GEMV / MoE-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  The product (chimere_amd/, libchimere_hip.so) never links or calls it.
 *
 * Block formats (byte-exact with ggml / the reference):
 *   Q8_0  34 B / 32 elem : [f16 d][i8 q[32]]                 gguf_loader.rs:793-837
 *   Q4_0  18 B / 32 elem : [f16 d][u8 nib[16]] lo=j, hi=j+16 gguf_loader.rs:752-772
 *   Q8_1  36 B / 32 elem : [f16 d][f16 s][i8 q[32]]          chimere_kernels.cu:1495-1523
 *   IQ3_S 110 B / 256 elem: [f16 d][qs 64][qh 8][signs 32][scales 4]
 *                                                           gguf_loader.rs:1008-1142
 *   Q4_K  144 B / 256    : [f16 d][f16 dmin][scales 12][qs 128]   gguf_loader.rs:1265-1330
 *   Q5_K  176 B / 256    : [f16 d][f16 dmin][scales 12][qh 32][qs 128]  :1165-1263
 *   Q6_K  210 B / 256    : [ql 128][qh 64][i8 scales 16][f16 d]   gguf_loader.rs:839-917
 *   MXFP4  17 B / 32     : [E8M0 e][u8 nib[16]] lo=j, hi=j+16     (ggml layout, see oracle.c)
 * Type ids follow ggml's enum: Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13,
 * Q6_K = 14, IQ3_S = 21, MXFP4 = 39.
 *
 * Canonical fp32 order ("L,G order") of a quantized row dot product:
 *   per 32-element block b (IQ3_S: sub-block b = 8*superblock + ib):
 *     sumi_b  = exact int32 block dot (IQ3_S: times (1 + 2*scale))
 *     scale_b = f32(d_w) * f32(d_x)                  (one rounding)
 *   slot j in [0,L) accumulates the blocks with (b / G) % L == j, ascending b:
 *     acc_j = fmaf(scale_b, (float)sumi_b, acc_j)    starting from +0.0f
 *     Q4_K / Q5_K then: acc_j = fmaf(-(f32(dmin)*f32(d_x)), (float)(m_b * sum q_x), acc_j)
 *     (their sumi_b = sc_b * sum q*q_x; Q6_K's = sc_lo*sum_lo + sc_hi*sum_hi of q-32;
 *      MXFP4's scale_b = 2^(e-128) * f32(d_x))
 *   then a halving tree: for m = L/2 .. 1: acc_i += acc_{i+m} (i < m); y = acc_0.
 * The GPU kernels document the (L, G) they use; the oracle reproduces that
 * order so that fp32 outputs (and hence every re-quantized intermediate)
 * are bit-identical.
 */
#ifndef CHIMERE_ORACLE_H
#define CHIMERE_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_IQ3_S = 21, ORC_MXFP4 = 39 };
/* Not a ggml type: Q4_0 blocks with ggml's block term (the "s-form")
 * d_w * (sum(nib * q_x) * d_x - 8 * s_x), s_x = f32 of the Q8_1 block's f16
 * sum of x, evaluated as inner = fmaf((float)sum, d_x, -(8 * s_x)),
 * acc = fmaf(d_w, inner, acc); sum uses the unsigned nibbles. */
enum { ORC_Q4_0_SFORM = 102 };

uint16_t orc_f32_to_f16(float x);
float    orc_f16_to_f32(uint16_t h);
float    orc_exp(float x);
/* every float in [lo, hi] <= 0: count of monotonicity violations, their
 * largest size in ulps, worst relative error against libm exp (x >= -86) */
int64_t  orc_exp_scan(float lo, float hi, int *max_step, double *max_rel);
float    orc_silu(float g);

int64_t  orc_row_bytes(int type, int64_t ncols);

/* Q8_1 (ggml semantics).  nrows rows of ncols floats (row stride ncols);
 * each output row is ncols_padded/32 blocks (elements >= ncols read as 0). */
void orc_quantize_q8_1(const float *x, int64_t ncols, int64_t ncols_padded,
                       int64_t nrows, uint8_t *out);
/* weight quantizers; n multiple of 32 (IQ3_S: 256) */
void orc_quantize_q8_0(const float *x, int64_t n, uint8_t *out);
void orc_quantize_q4_0(const float *x, int64_t n, uint8_t *out);
void orc_quantize_iq3_s(const float *x, int64_t n, uint8_t *out);
void orc_dequantize(int type, const uint8_t *w, int64_t n, float *out);

/* int32 block dots: out[r * (ncols/32) + b] */
void orc_block_dots(int type, const uint8_t *W, const uint8_t *xq,
                    int ncols, int nrows, int32_t *out);

/* y[t*nrows + r] = row r of W . token t of xq (token stride xq_stride bytes) */
void orc_gemv(int type, const uint8_t *W, const uint8_t *xq, int64_t xq_stride,
              float *y, int ncols, int nrows, int ntok, int L, int G, int nthreads);

/* reference CPU path for Q8_0 (f64 accumulation, unquantized x): ffi/src/lib.rs:107-154 */
void orc_gemv_q8_0_f64(const uint8_t *W, const float *x, float *y,
                       int ncols, int nrows);

/* f32 router GEMV in the order of elementwise.rs:186-221 (256 slots, halving tree) */
void orc_router(const float *Wr, const float *x, float *logits, int E, int H);
/* softmax + top-k + renorm, chimere_kernels.cu:1150-1223 */
void orc_topk_softmax(const float *logits, int E, int K, int32_t *idx, float *w);

typedef struct {
    int H, F, E, K, M;
    int exp_type, sh_type;                 /* ggml type ids; sh_type < 0: no shared expert */
    const float   *router;                 /* [E*H] f32 */
    const float   *logit_bias;             /* [E] or NULL, added to router logits */
    const uint8_t *gate, *up, *down;       /* stacked experts */
    int64_t        stride_gate, stride_up, stride_down;  /* bytes per expert */
    const uint8_t *sh_gate, *sh_up, *sh_down;
    const float   *sh_gate_w;              /* [H] or NULL (gate = 1) */
    int L, G;                              /* row-dot order */
} orc_moe_params;

/* Full MoE FFN layer for M tokens.  x [M*H], out [M*H]; optional debug
 * outputs (may be NULL): ids [M*K], wts [M*K]. */
void orc_moe(const orc_moe_params *p, const float *x, float *out,
             int32_t *ids, float *wts, int nthreads);

/* ncmoe CPU expert path (moe_ffn.rs:1507-1591, ffi/ggml_iq3s_gemv.c): Q8_K
 * activations (296-byte blocks), IQ3_S x Q8_K dots, the one-token expert loop. */
/* fused MoE on f32 activations, IQ3_S experts (the library's fixed order):
 * out[r] += sum_k wts[k] * (D_{ids[k]} (silu(G x) * (U x)))[r] */
void orc_fused_moe_iq3s(const float *x, const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                        const int32_t *ids, const float *wts, float *out, int H, int F,
                        int64_t bg, int64_t bu, int64_t bd, int K);
void orc_quantize_q8_K(const float *x, int64_t k, uint8_t *out);
float orc_vec_dot_iq3s_q8K(int n, const uint8_t *w, const uint8_t *y);
void orc_gemv_iq3s_q8K(const uint8_t *W, const float *x, float *y, int nrows, int ncols);
void orc_ncmoe(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t sg, int64_t su, int64_t sd,
               const int32_t *ids, const float *wts, int K, const float *x, float *out, int H, int F);
/* orc_moe with the routed experts on the ncmoe CPU path (IQ3_S experts) */
void orc_moe_ncmoe(const orc_moe_params *p, const float *x, float *out, int32_t *ids, float *wts, int nthreads);

/* CPU baseline (cpu_path.c): the reference's CPU path structure with AVX2
 * vec_dots (Q8_0 / Q4_0 / IQ3_S weights, Q8_1 activations), OpenMP
 * row-parallel with nthreads threads; agrees with the oracle to the fp32
 * tolerance, not bit for bit. */
void cpb_gemv(int type, const uint8_t *W, const uint8_t *xq, float *y, int ncols, int nrows, int nthreads);
void cpb_moe(const orc_moe_params *p, const float *x, float *out, int32_t *ids, float *wts, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
