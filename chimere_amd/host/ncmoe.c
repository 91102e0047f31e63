/* CPU expert path ("ncmoe"): routed experts whose IQ3_S weights stay in host
 * memory, evaluated on the host cores for one token while the router, the
 * shared expert and everything else run on the GPU.
 *
 * Replaces the reference's ggml wrapper (cs/ffi/ggml_iq3s_gemv.c:33-127,
 * declarations cs/ffi/ggml_iq3s_gemv.h:19-64) under the same exported names,
 * and the per-token expert loop of cs/src/qwen35_model/moe_ffn.rs:1507-1591
 * as one call (chimere_ncmoe_experts).
 *
 * Arithmetic:
 *   - Q8_K activations (296-byte blocks: f32 d, f32 sum, int8 q[256],
 *     int16 bsums[16]).  Per 256 values: m = the first value of largest
 *     magnitude; m == 0 -> a zero block; else iscale = -127 / m,
 *     q = min(127, round-half-even(iscale * x)), d = 1 / iscale,
 *     sum = d * sum(q), bsums = sums of 16 consecutive q.
 *   - IQ3_S x Q8_K dot: per super-block the exact integer
 *     sum_ib (1 + 2 s_ib) * sum_e (+-grid level_e) * q_e, then in super-block
 *     order acc = fmaf(f32(d_w) * d_y, (float)isum, acc).  The integer part
 *     runs in AVX2 (maddubs/madd: every partial fits in int16/int32) or a
 *     scalar loop; both give the same integer, so the float result does not
 *     depend on the instruction set or the thread count.
 *   - expert loop: h = (g / (1 + expf(-g))) * u in f32, down = W_d h with
 *     h quantized to Q8_K, out += w_k * down in the order of the ids.
 * Built with -ffp-contract=off: every fused multiply-add is an explicit
 * fmaf(). */
#include "chimere_cpu.h"

#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../csrc/iq3s_grid.inc"

#define IQ3S_BYTES 110
#define Q8K_BYTES 296
#define QK 256

static const uint32_t k_grid[512] = CHIMERE_IQ3S_GRID_INIT;

static inline float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {               /* subnormal: normalise */
            int s = 0;
            while (!(m & 0x400u)) { m <<= 1; s++; }
            bits = sign | ((uint32_t)(113 - s) << 23) | ((m & 0x3FFu) << 13);
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* --------------------------------------------------------------- Q8_K */

static void quantize_q8K(const float *x, uint8_t *y, int64_t k) {
    for (int64_t b = 0; b < k / QK; b++) {
        const float *v = x + b * QK;
        uint8_t *o = y + b * Q8K_BYTES;
        float amax = 0.0f, m = 0.0f;
        for (int j = 0; j < QK; j++) {
            const float a = fabsf(v[j]);
            if (a > amax) { amax = a; m = v[j]; }
        }
        if (amax == 0.0f) {
            memset(o, 0, Q8K_BYTES);
            continue;
        }
        const float iscale = -127.0f / m;
        int8_t q[QK];
        int32_t tot = 0;
        for (int j = 0; j < QK; j++) {
            const float t = rintf(iscale * v[j]);   /* current rounding mode: nearest-even */
            q[j] = (int8_t)(t < 127.0f ? (int)t : 127);
        }
        int16_t bs[16];
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) s += q[16 * g + j];
            bs[g] = (int16_t)s;
            tot += s;
        }
        const float d = 1.0f / iscale, sum = d * (float)tot;
        memcpy(o, &d, 4);
        memcpy(o + 4, &sum, 4);
        memcpy(o + 8, q, QK);
        memcpy(o + 8 + QK, bs, 32);
    }
}

/* ------------------------------------------------- IQ3_S super-block sums */

/* exact integer sum of one 110-byte super-block against 256 int8 values */
static int32_t sb_isum_scalar(const uint8_t *w, const int8_t *q) {
    int32_t tot = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t *qs = w + 2 + 8 * ib, *sg = w + 74 + 4 * ib;
        const int qh = w[66 + ib];
        int32_t s = 0;
        for (int p = 0; p < 8; p++) {            /* 8 groups of 4 values */
            const uint32_t gv = k_grid[qs[p] | (((qh >> p) & 1) << 8)];
            const int sb = sg[p >> 1] >> (4 * (p & 1));
            for (int j = 0; j < 4; j++) {
                const int lv = (int)((gv >> (8 * j)) & 0xFFu);
                const int v = q[32 * ib + 4 * p + j];
                /* the sign flips the int8 activation, wrapping as the SIMD
                 * paths' byte negation does (-(-128) stays -128) */
                s += lv * ((sb >> j) & 1 ? (int)(int8_t)(uint8_t)(-v) : v);
            }
        }
        tot += s * (1 + 2 * ((w[106 + ib / 2] >> (4 * (ib & 1))) & 0xF));
    }
    return tot;
}

/* the 8 codebook entries of a sub-block: 9-bit indices qs[p] | (qh bit p) << 8 */
__attribute__((target("avx2"))) static inline __m256i sub_levels(const uint8_t *qs, int qh) {
    uint64_t q8;
    memcpy(&q8, qs, 8);
    const __m256i lo = _mm256_cvtepu8_epi32(_mm_cvtsi64_si128((long long)q8));
    const __m256i bit = _mm256_setr_epi32(1, 2, 4, 8, 16, 32, 64, 128);
    const __m256i hi = _mm256_and_si256(_mm256_cmpeq_epi32(_mm256_and_si256(_mm256_set1_epi32(qh), bit), bit),
                                        _mm256_set1_epi32(256));
    return _mm256_i32gather_epi32((const int *)k_grid, _mm256_or_si256(lo, hi), 4);
}

/* +1 / -1 per byte from the 32 sign bits of a sub-block */
__attribute__((target("avx2"))) static inline __m256i sub_signs(const uint8_t *sg) {
    uint32_t bits;
    memcpy(&bits, sg, 4);
    const __m256i rep = _mm256_shuffle_epi8(_mm256_set1_epi32((int)bits),
                                            _mm256_setr_epi8(0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1,
                                                             2, 2, 2, 2, 2, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3, 3));
    const __m256i bit = _mm256_set1_epi64x((long long)0x8040201008040201ULL);
    const __m256i neg = _mm256_cmpeq_epi8(_mm256_and_si256(rep, bit), bit);
    return _mm256_or_si256(neg, _mm256_set1_epi8(1));
}

__attribute__((target("avx2"))) static int32_t sb_isum_avx2(const uint8_t *w, const int8_t *q) {
    __m256i acc = _mm256_setzero_si256();
    for (int ib = 0; ib < 8; ib += 2) {
        const __m256i l0 = sub_levels(w + 2 + 8 * ib, w[66 + ib]);
        const __m256i l1 = sub_levels(w + 2 + 8 * ib + 8, w[67 + ib]);
        const __m256i q0 = _mm256_sign_epi8(_mm256_loadu_si256((const __m256i *)(q + 32 * ib)), sub_signs(w + 74 + 4 * ib));
        const __m256i q1 = _mm256_sign_epi8(_mm256_loadu_si256((const __m256i *)(q + 32 * ib + 32)), sub_signs(w + 78 + 4 * ib));
        /* unsigned levels (<= 15) x signed q (|q| <= 127): pair sums fit int16 */
        const __m256i p0 = _mm256_maddubs_epi16(l0, q0), p1 = _mm256_maddubs_epi16(l1, q1);
        const int sc = w[106 + ib / 2];
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p0, _mm256_set1_epi16((short)(1 + 2 * (sc & 0xF)))));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p1, _mm256_set1_epi16((short)(1 + 2 * (sc >> 4)))));
    }
    const __m128i s = _mm_add_epi32(_mm256_castsi256_si128(acc), _mm256_extracti128_si256(acc, 1));
    const __m128i s2 = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    return _mm_cvtsi128_si32(_mm_add_epi32(s2, _mm_shuffle_epi32(s2, 0xB1)));
}

/* AVX-512 (F + BW): two sub-blocks (64 weights) per step.  The 16 codebook
 * entries come from one 16-lane gather (the high index bits set by a lane
 * mask test), the 64 sign bits negate the activations as a byte mask, and
 * the two sub-blocks' multipliers sit in the low / high 256 bits of the
 * multiplier vector. */
__attribute__((target("avx512f,avx512bw"))) static int32_t sb_isum_avx512(const uint8_t *w, const int8_t *q) {
    const __m512i lane_bit = _mm512_setr_epi32(1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192,
                                               16384, 32768);
    __m512i acc = _mm512_setzero_si512();
    for (int ib = 0; ib < 8; ib += 2) {
        const __m512i lo = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i *)(w + 2 + 8 * ib)));
        const int qh = w[66 + ib] | (w[67 + ib] << 8);
        const __mmask16 hb = _mm512_test_epi32_mask(_mm512_set1_epi32(qh), lane_bit);
        const __m512i idx = _mm512_mask_or_epi32(lo, hb, lo, _mm512_set1_epi32(256));
        const __m512i lev = _mm512_i32gather_epi32(idx, (const void *)k_grid, 4);
        uint64_t sg;
        memcpy(&sg, w + 74 + 4 * ib, 8);
        const __m512i qv = _mm512_loadu_si512((const void *)(q + 32 * ib));
        const __m512i qs = _mm512_mask_sub_epi8(qv, (__mmask64)sg, _mm512_setzero_si512(), qv);
        const int sc = w[106 + ib / 2];
        const __m512i mult = _mm512_mask_set1_epi16(_mm512_set1_epi16((short)(1 + 2 * (sc & 0xF))), (__mmask32)0xFFFF0000u,
                                                    (short)(1 + 2 * (sc >> 4)));
        acc = _mm512_add_epi32(acc, _mm512_madd_epi16(_mm512_maddubs_epi16(lev, qs), mult));
    }
    return _mm512_reduce_add_epi32(acc);
}

typedef int32_t (*isum_fn)(const uint8_t *, const int8_t *);
static isum_fn g_isum;

/* chosen once at load time, before any caller thread exists: AVX-512, else
 * AVX2, else the portable loop (all give the same integers);
 * CHIMERE_CPU_NO_AVX512=1 / CHIMERE_CPU_PORTABLE=1 step down (for tests) */
__attribute__((constructor)) static void choose_isum(void) {
    __builtin_cpu_init();
    const char *e = getenv("CHIMERE_CPU_PORTABLE");
    const int portable = e && e[0] == '1';
    const char *e2 = getenv("CHIMERE_CPU_NO_AVX512");
    if (!portable && !(e2 && e2[0] == '1') && __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw"))
        g_isum = sb_isum_avx512;
    else if (!portable && __builtin_cpu_supports("avx2"))
        g_isum = sb_isum_avx2;
    else
        g_isum = sb_isum_scalar;
}

static inline isum_fn pick_isum(void) { return g_isum; }

static inline float row_dot(isum_fn isum, int n, const uint8_t *w, const uint8_t *y) {
    float acc = 0.0f;
    for (int b = 0; b < n / QK; b++) {
        const uint8_t *wb = w + (int64_t)b * IQ3S_BYTES, *yb = y + (int64_t)b * Q8K_BYTES;
        float dy;
        memcpy(&dy, yb, 4);
        const int32_t s = isum(wb, (const int8_t *)(yb + 8));
        acc = fmaf(half_to_float((uint16_t)(wb[0] | (wb[1] << 8))) * dy, (float)s, acc);
    }
    return acc;
}

/* ------------------------------------------------------------ ggml_ffi_* */

void ggml_ffi_quantize_q8_K(const float *x, void *y, int64_t k) { quantize_q8K(x, (uint8_t *)y, k); }

void ggml_ffi_vec_dot_iq3s_q8K(int n, float *s, const void *vx, const void *vy) {
    *s = row_dot(pick_isum(), n, (const uint8_t *)vx, (const uint8_t *)vy);
}

static void gemv_rows(const uint8_t *w, const uint8_t *xq, float *y, int nrows, int ncols, int nthreads) {
    const isum_fn isum = pick_isum();
    const int64_t rb = (int64_t)(ncols / QK) * IQ3S_BYTES;
#ifdef _OPENMP
    if (nthreads != 1) {
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : omp_get_max_threads()) schedule(static)
        for (int r = 0; r < nrows; r++) y[r] = row_dot(isum, ncols, w + r * rb, xq);
        return;
    }
#else
    (void)nthreads;
#endif
    for (int r = 0; r < nrows; r++) y[r] = row_dot(isum, ncols, w + r * rb, xq);
}

void ggml_ffi_gemv_iq3s(const void *w_iq3s, const float *x_f32, float *y_f32, int nrows, int ncols) {
    ggml_ffi_gemv_iq3s_parallel(w_iq3s, x_f32, y_f32, nrows, ncols, 1);
}

void ggml_ffi_gemv_iq3s_parallel(const void *w_iq3s, const float *x_f32, float *y_f32, int nrows, int ncols,
                                 int nthreads) {
    uint8_t *xq = (uint8_t *)malloc((size_t)(ncols / QK) * Q8K_BYTES + 1);
    if (!xq) return;
    quantize_q8K(x_f32, xq, ncols);
    gemv_rows((const uint8_t *)w_iq3s, xq, y_f32, nrows, ncols, nthreads);
    free(xq);
}

size_t ggml_ffi_iq3s_row_bytes(int ncols) { return (size_t)(ncols / QK) * IQ3S_BYTES; }

size_t ggml_ffi_q8k_row_bytes(int ncols) { return (size_t)(ncols / QK) * Q8K_BYTES; }

/* ------------------------------------------------------ the expert loop */

int chimere_ncmoe_experts(const void *gate_exps, const void *up_exps, const void *down_exps, size_t expert_bytes_gate,
                          size_t expert_bytes_up, size_t expert_bytes_down, const int32_t *ids, const float *weights,
                          int top_k, const float *hidden, float *combined, int hidden_size, int expert_ffn,
                          int n_experts, int nthreads) {
    if (!gate_exps || !up_exps || !down_exps || !ids || !weights || !hidden || !combined) return CHIMERE_CPU_EINVAL;
    if (top_k < 1 || top_k > 64 || hidden_size <= 0 || expert_ffn <= 0 || hidden_size % QK || expert_ffn % QK)
        return CHIMERE_CPU_EINVAL;
    if (expert_bytes_gate < (size_t)expert_ffn * ggml_ffi_iq3s_row_bytes(hidden_size) ||
        expert_bytes_up < (size_t)expert_ffn * ggml_ffi_iq3s_row_bytes(hidden_size) ||
        expert_bytes_down < (size_t)hidden_size * ggml_ffi_iq3s_row_bytes(expert_ffn))
        return CHIMERE_CPU_EINVAL;
    for (int k = 0; k < top_k; k++)
        if (ids[k] < 0 || ids[k] >= n_experts) return CHIMERE_CPU_EINVAL;

    const int H = hidden_size, F = expert_ffn, K = top_k;
    const int64_t xb = (int64_t)(H / QK) * Q8K_BYTES, hb = (int64_t)(F / QK) * Q8K_BYTES;
    const int64_t rbh = (int64_t)(H / QK) * IQ3S_BYTES, rbf = (int64_t)(F / QK) * IQ3S_BYTES;
    uint8_t *xq = (uint8_t *)malloc((size_t)(xb + (int64_t)K * hb));
    float *gu = (float *)malloc(sizeof(float) * (size_t)(2 * K * F + K * H));
    if (!xq || !gu) {
        free(xq);
        free(gu);
        return CHIMERE_CPU_ENOMEM;
    }
    uint8_t *hq = xq + xb;
    float *dn = gu + 2 * (int64_t)K * F;
    const uint8_t *G = (const uint8_t *)gate_exps, *U = (const uint8_t *)up_exps, *D = (const uint8_t *)down_exps;
    const isum_fn isum = pick_isum();
    quantize_q8K(hidden, xq, H);
#ifdef _OPENMP
    const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        /* gate and up rows of every selected expert: they all read x alone */
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int r = 0; r < 2 * K * F; r++) {
            const int k = r / (2 * F), rr = r % (2 * F);
            const uint8_t *w = rr < F ? G + (size_t)ids[k] * expert_bytes_gate + (int64_t)rr * rbh
                                      : U + (size_t)ids[k] * expert_bytes_up + (int64_t)(rr - F) * rbh;
            gu[r] = row_dot(isum, H, w, xq);
        }
        /* SwiGLU per expert, then its Q8_K intermediate */
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int k = 0; k < K; k++) {
            float *g = gu + 2 * (int64_t)k * F;
            const float *u = g + F;
            for (int i = 0; i < F; i++) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
            quantize_q8K(g, hq + k * hb, F);
        }
        /* down rows of every selected expert */
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int r = 0; r < K * H; r++) {
            const int k = r / H, rr = r % H;
            dn[r] = row_dot(isum, F, D + (size_t)ids[k] * expert_bytes_down + (int64_t)rr * rbf, hq + k * hb);
        }
        /* weighted sum in the order of the ids */
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int i = 0; i < H; i++) {
            float s = 0.0f;
            for (int k = 0; k < K; k++) s = s + weights[k] * dn[(int64_t)k * H + i];
            combined[i] = s;
        }
    }
    free(xq);
    free(gu);
    return CHIMERE_CPU_OK;
}

int chimere_cpu_isa(void) { return pick_isum() == sb_isum_avx512 ? 2 : pick_isum() == sb_isum_avx2 ? 1 : 0; }
