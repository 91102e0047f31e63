/*
 * cpu_path.c -- the CPU baseline: a restatement, with AVX2, of the
 * reference's CPU GEMV path (cs/ffi/ggml_iq3s_gemv.c:84-127: activations
 * quantized once per call, then an OpenMP `parallel for schedule(static)`
 * over the rows, one SIMD vec_dot per row) and of the decode MoE sequence it
 * serves (cs/src/qwen35_model/moe_ffn.rs:1185-1384, 1507-1591 per token).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): bench.py times it as the reported
 * CPU baseline and tests/ check it against the oracle; the product never
 * loads it.
 *
 * Differences from the reference's CPU path, on purpose: activations use
 * the Q8_1 blocks of the GPU contract (the reference's CPU IQ3_S path uses
 * ggml's Q8_K, 256-element blocks), so its int32 block dots are the oracle's;
 * the fp32 combination of a row is ggml's (8-lane partial sums scaled per
 * block, one horizontal sum per row), so outputs agree with the oracle to
 * the fp32 tolerance (1e-5 of ||y|| for Q8_0 / Q4_0, 1e-4 for IQ3_S), not
 * bit for bit.
 */
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

#include "iq3s_grid.inc"

static inline float f16f(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* 32 signed int8 weights w times the Q8_1 block's 32 int8 q: 8 int32 lanes */
static inline __m256i dot32(__m256i w, __m256i q) {
    const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(q, w));
    return _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
}

static float row_q8_0(const uint8_t *w, const uint8_t *xq, int nb) {
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < nb; b++) {
        const uint8_t *wb = w + 34 * b, *xb = xq + 36 * b;
        const __m256i p = dot32(_mm256_loadu_si256((const __m256i *)(wb + 2)),
                                _mm256_loadu_si256((const __m256i *)(xb + 4)));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(f16f(wb) * f16f(xb)), _mm256_cvtepi32_ps(p), acc);
    }
    return hsum8(acc);
}

static float row_q4_0(const uint8_t *w, const uint8_t *xq, int nb) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i m4 = _mm256_set1_epi8(0x0F), e8 = _mm256_set1_epi8(8);
    for (int b = 0; b < nb; b++) {
        const uint8_t *wb = w + 18 * b, *xb = xq + 36 * b;
        const __m128i nib = _mm_loadu_si128((const __m128i *)(wb + 2));
        /* elements 0..15 = low nibbles, 16..31 = high nibbles */
        const __m256i v = _mm256_and_si256(_mm256_set_m128i(_mm_srli_epi16(nib, 4), nib), m4);
        const __m256i p = dot32(_mm256_sub_epi8(v, e8), _mm256_loadu_si256((const __m256i *)(xb + 4)));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(f16f(wb) * f16f(xb)), _mm256_cvtepi32_ps(p), acc);
    }
    return hsum8(acc);
}

/* IQ3_S: per 32-element sub-block, 8 codebook words and 32 sign bits give
 * the signed levels; the int dot is scaled by (1 + 2 s) and d * d_x. */
static float row_iq3_s(const uint8_t *w, const uint8_t *xq, int nsb) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i bits = _mm256_set1_epi64x((long long)0x8040201008040201ULL);
    const __m256i spread = _mm256_set_epi64x(0x0303030303030303LL, 0x0202020202020202LL,
                                             0x0101010101010101LL, 0x0000000000000000LL);
    for (int s = 0; s < nsb; s++) {
        const uint8_t *sb = w + 110 * s;
        const float d = f16f(sb);
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t *qs = sb + 2 + 8 * ib, qh = sb[66 + ib], *sg = sb + 74 + 4 * ib;
            const __m256i g = _mm256_set_epi32(
                (int)orc_iq3s_grid[qs[7] | ((qh << 1) & 256)], (int)orc_iq3s_grid[qs[6] | ((qh << 2) & 256)],
                (int)orc_iq3s_grid[qs[5] | ((qh << 3) & 256)], (int)orc_iq3s_grid[qs[4] | ((qh << 4) & 256)],
                (int)orc_iq3s_grid[qs[3] | ((qh << 5) & 256)], (int)orc_iq3s_grid[qs[2] | ((qh << 6) & 256)],
                (int)orc_iq3s_grid[qs[1] | ((qh << 7) & 256)], (int)orc_iq3s_grid[qs[0] | ((qh << 8) & 256)]);
            /* byte k of the sign word selects bit (k % 8) of sign byte k / 8 */
            uint32_t s32;
            memcpy(&s32, sg, 4);
            const __m256i sb8 = _mm256_shuffle_epi8(_mm256_set1_epi32((int)s32), spread);
            const __m256i neg = _mm256_cmpeq_epi8(_mm256_and_si256(sb8, bits), bits);
            const __m256i v = _mm256_sub_epi8(_mm256_xor_si256(g, neg), neg);
            const uint8_t *xb = xq + 36 * (8 * s + ib);
            const __m256i p = dot32(v, _mm256_loadu_si256((const __m256i *)(xb + 4)));
            const int mult = 1 + 2 * ((sb[106 + ib / 2] >> (4 * (ib & 1))) & 15);
            acc = _mm256_fmadd_ps(_mm256_set1_ps(d * f16f(xb) * (float)mult), _mm256_cvtepi32_ps(p), acc);
        }
    }
    return hsum8(acc);
}

static inline float row_dot(int type, const uint8_t *w, const uint8_t *xq, int ncols) {
    switch (type) {
    case ORC_Q8_0: return row_q8_0(w, xq, ncols / 32);
    case ORC_Q4_0: return row_q4_0(w, xq, ncols / 32);
    default: return row_iq3_s(w, xq, ncols / 256);
    }
}

void cpb_gemv(int type, const uint8_t *W, const uint8_t *xq, float *y, int ncols, int nrows, int nthreads) {
    const int64_t rb = orc_row_bytes(type, ncols);
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int r = 0; r < nrows; r++) y[r] = row_dot(type, W + (int64_t)r * rb, xq, ncols);
}

static float dot_f32(const float *a, const float *b, int n) {
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), s1);
    }
    float t = hsum8(_mm256_add_ps(s0, s1));
    for (; i < n; i++) t += a[i] * b[i];
    return t;
}

/* One or more tokens through the decode MoE sequence, one token at a time as
 * the reference does: router (row-parallel f32 dots) -> softmax/top-k ->
 * Q8_1(x) -> gate/up rows of every selected expert and the shared expert
 * (one parallel loop) -> silu(gate) * up -> Q8_1(h) -> down rows (one
 * parallel loop) -> k-ordered weighted sum + shared expert. */
void cpb_moe(const orc_moe_params *p, const float *x, float *out, int32_t *ids, float *wts, int nthreads) {
    const int H = p->H, F = p->F, E = p->E, K = p->K;
    const int NP = K + (p->sh_type >= 0 ? 1 : 0);
    const int64_t xqb = (H + 511) / 512 * 512 / 32 * 36, hqb = (F + 511) / 512 * 512 / 32 * 36;
    float *logits = malloc(sizeof(float) * E), *gu = malloc(sizeof(float) * NP * 2 * F);
    float *dn = malloc(sizeof(float) * NP * H);
    uint8_t *xq = malloc(xqb), *hq = malloc(hqb * NP);
    float *h = malloc(sizeof(float) * F);
    int32_t id[1024];
    float w[1024];
    for (int t = 0; t < p->M; t++) {
        const float *xt = x + (int64_t)t * H;
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (int e = 0; e < E; e++) logits[e] = dot_f32(p->router + (int64_t)e * H, xt, H);
        if (p->logit_bias)
            for (int e = 0; e < E; e++) logits[e] += p->logit_bias[e];
        orc_topk_softmax(logits, E, K, id, w);
        if (ids) memcpy(ids + (int64_t)t * K, id, sizeof(int32_t) * K);
        if (wts) memcpy(wts + (int64_t)t * K, w, sizeof(float) * K);
        orc_quantize_q8_1(xt, H, (H + 511) / 512 * 512, 1, xq);
        const int64_t rbH = orc_row_bytes(p->exp_type, H), rbHs = p->sh_type >= 0 ? orc_row_bytes(p->sh_type, H) : 0;
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (int i = 0; i < NP * 2 * F; i++) {
            const int k = i / (2 * F), r = i % (2 * F);
            const uint8_t *m;
            int type;
            if (k < K) {
                type = p->exp_type;
                m = (r < F ? p->gate + id[k] * p->stride_gate : p->up + id[k] * p->stride_up) + (int64_t)(r % F) * rbH;
            } else {
                type = p->sh_type;
                m = (r < F ? p->sh_gate : p->sh_up) + (int64_t)(r % F) * rbHs;
            }
            gu[i] = row_dot(type, m, xq, H);
        }
        for (int k = 0; k < NP; k++) {
            for (int f = 0; f < F; f++) h[f] = orc_silu(gu[k * 2 * F + f]) * gu[k * 2 * F + F + f];
            orc_quantize_q8_1(h, F, (F + 511) / 512 * 512, 1, hq + k * hqb);
        }
        const int64_t rbF = orc_row_bytes(p->exp_type, F), rbFs = p->sh_type >= 0 ? orc_row_bytes(p->sh_type, F) : 0;
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (int i = 0; i < NP * H; i++) {
            const int k = i / H, r = i % H;
            if (k < K) dn[i] = row_dot(p->exp_type, p->down + id[k] * p->stride_down + (int64_t)r * rbF, hq + k * hqb, F);
            else dn[i] = row_dot(p->sh_type, p->sh_down + (int64_t)r * rbFs, hq + k * hqb, F);
        }
        float *o = out + (int64_t)t * H;
        float sc = 1.0f;
        if (p->sh_type >= 0 && p->sh_gate_w) sc = 1.0f / (1.0f + orc_exp(-dot_f32(p->sh_gate_w, xt, H)));
        for (int i = 0; i < H; i++) {
            float a = 0.0f;
            for (int k = 0; k < K; k++) a = fmaf(w[k], dn[k * H + i], a);
            o[i] = p->sh_type >= 0 ? fmaf(dn[K * H + i], sc, a) : a;
        }
    }
    free(logits); free(gu); free(dn); free(xq); free(hq); free(h);
}
