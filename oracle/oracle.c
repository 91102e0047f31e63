/*
 * oracle.c -- CPU restatement of the reference's quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with -ffp-contract=off
 * so that every fused multiply-add below is an explicit fmaf(); together
 * with IEEE add/mul/div and the deterministic exponential orc_exp() this
 * reproduces the HIP kernels' arithmetic bit for bit.
 *
 * Reference citations (paths relative to the reference repository root,
 * cs/ = chimere-server/):
 *   Q8_1 quantizer      cs/kernels/chimere_kernels.cu:1495-1523 (ggml port),
 *                       warp butterfly order :1327-1333
 *   Q8_0 quantizer      cs/src/kernels/kv_q8_0.rs:49-89
 *   Q8_0 dot            cs/src/kernels/gemv_q8_0.rs:230-255
 *   Q4_0 layout         cs/src/gguf_loader.rs:752-772
 *   IQ3_S layout/dot    cs/src/gguf_loader.rs:1008-1142, cs/src/kernels/iq3s_gemv.rs:292-352
 *   router GEMV         cs/src/kernels/elementwise.rs:186-221
 *   top-k softmax       cs/kernels/chimere_kernels.cu:1150-1223
 *   SiLU*up             cs/src/kernels/fused_ops.rs:34-45
 *   weighted combine    cs/src/kernels/fused_ops.rs:364-378
 *   shared-expert gate  cs/src/scratch_pool.rs:243-277
 *   MoE op order        cs/src/qwen35_model/moe_ffn.rs:1081-1768
 *   f64 Q8_0 CPU path   cs/ffi/src/lib.rs:107-154
 *   Q4_K / Q5_K layout  cs/src/gguf_loader.rs:1145-1330 (get_scale_min_k4 :1150-1163)
 *   Q6_K layout         cs/src/gguf_loader.rs:839-917
 *   K-quant dot ints    cs/kernels/chimere_kernels.cu:1344-1440 (sc * sum q*q_x and
 *                       m * sum q_x, both exact integers)
 *   MXFP4               entry points only (cs/ffi/ggml_cuda_gemv.cu:407-460); the
 *                       block layout is ggml's published one (no code in the
 *                       reference tree): [E8M0 e][16 B nibbles], level table
 *                       {0,1,2,3,4,6,8,12} (E2M1 doubled), sign = bit 3,
 *                       scale 2^(e-128).
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "iq3s_grid.inc"

/* ------------------------------------------------------------------ f16 */

uint16_t orc_f32_to_f16(float x) {
    /* IEEE binary32 -> binary16, round to nearest even, subnormals kept. */
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ex = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;                   /* 14..24 */
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;   /* may carry into exponent: correct */
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t u;
    if (ex == 0) {
        float f = (float)man * 0x1p-24f;
        memcpy(&u, &f, 4);
        u |= sign;
    } else if (ex == 31) {
        u = sign | 0x7F800000u | (man << 13);
    } else {
        u = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* ------------------------------------------------------------------ exp */

/* Deterministic exp: Cody-Waite reduction x = n*ln2 + r with a two-part ln2
 * (high part 0x1.62e4p-1 has trailing zero bits), then the degree-7 Taylor
 * polynomial of e^r (|r| <= ln2/2, truncation error < 6e-9 relative) in
 * Horner form, then scaling by 2^n.  Inputs below -86 return 0 (so no
 * subnormal results), above 88.7228 return +inf.  The HIP library uses the
 * same operation sequence, so results agree bit for bit. */
float orc_exp(float x) {
    if (x != x) return x;
    if (x > 88.72283905f) return INFINITY;
    if (x < -86.0f) return 0.0f;
    float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e4p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

float orc_silu(float g) { return g / (1.0f + orc_exp(-g)); }

/* Check of orc_exp over every float in [lo, hi] (lo <= hi <= 0): returns the
 * number of adjacent float pairs x < y with orc_exp(x) > orc_exp(y);
 * *max_step receives the largest such excess in units in the last place of
 * the result, *max_rel the largest |orc_exp(x) - e^x| / e^x over x >= -86
 * (the flush-to-zero bound), with e^x from libm's double exp. */
int64_t orc_exp_scan(float lo, float hi, int *max_step, double *max_rel) {
    uint32_t ulo, uhi;
    memcpy(&ulo, &lo, 4);
    memcpy(&uhi, &hi, 4);
    /* negative floats: bit patterns increase as values decrease */
    const uint32_t a = uhi == 0 ? 0x80000000u : uhi, b = ulo;   /* [a, b] covers hi down to lo */
    int64_t bad = 0;
    int step = 0;
    double worst = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : bad) reduction(max : worst, step)
    for (int64_t c = 0; c < 4096; c++) {
        const uint64_t n = (uint64_t)(b - a) + 1;
        const uint32_t s0 = a + (uint32_t)(n * (uint64_t)c / 4096), s1 = a + (uint32_t)(n * (uint64_t)(c + 1) / 4096);
        float prev_x;
        uint32_t u0 = s0;
        memcpy(&prev_x, &u0, 4);
        float prev = orc_exp(prev_x);
        /* walk from larger values (s0) to smaller ones: exp must not increase */
        for (uint32_t u = s0 + 1; u <= s1 && u <= b; u++) {
            float x;
            memcpy(&x, &u, 4);
            const float e = orc_exp(x);
            if (e > prev) {
                uint32_t ue, up;
                memcpy(&ue, &e, 4);
                memcpy(&up, &prev, 4);
                bad++;
                if ((int)(ue - up) > step) step = (int)(ue - up);
            }
            if (x >= -86.0f) {
                const double t = exp((double)x);
                const double r = fabs((double)e - t) / t;
                if (r > worst) worst = r;
            }
            prev = e;
        }
    }
    if (max_step) *max_step = step;
    if (max_rel) *max_rel = worst;
    return bad;
}

/* ------------------------------------------------------------- formats */

int64_t orc_row_bytes(int type, int64_t ncols) {
    switch (type) {
    case ORC_Q8_0: return ncols / 32 * 34;
    case ORC_Q4_0: case ORC_Q4_0_SFORM: return ncols / 32 * 18;
    case ORC_IQ3_S: return ncols / 256 * 110;
    case ORC_Q4_K: return ncols / 256 * 144;
    case ORC_Q5_K: return ncols / 256 * 176;
    case ORC_Q6_K: return ncols / 256 * 210;
    case ORC_MXFP4: return ncols / 32 * 17;
    default: return -1;
    }
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* Q8_1, ggml semantics (chimere_kernels.cu:1495-1523): per 32-block,
 * d = amax/127, q = amax==0 ? 0 : roundf(x/d), ds = (f16(d), f16(sum x)),
 * sum taken in the 32-lane xor-butterfly order (masks 16,8,4,2,1). */
static void q8_1_block(const float *v, uint8_t *o) {
    float amax = 0.0f, s[32], t[32];
    for (int i = 0; i < 32; i++) { float a = fabsf(v[i]); amax = a > amax ? a : amax; s[i] = v[i]; }
    for (int m = 16; m >= 1; m >>= 1) {
        for (int i = 0; i < 32; i++) t[i] = s[i] + s[i ^ m];
        memcpy(s, t, sizeof s);
    }
    float d = amax / 127.0f;
    for (int i = 0; i < 32; i++) o[4 + i] = (uint8_t)(int8_t)(amax == 0.0f ? 0 : (int)roundf(v[i] / d));
    wr16(o, orc_f32_to_f16(d));
    wr16(o + 2, orc_f32_to_f16(s[0]));
}

void orc_quantize_q8_1(const float *x, int64_t ncols, int64_t ncols_padded,
                       int64_t nrows, uint8_t *out) {
    int64_t nb = ncols_padded / 32;
    for (int64_t r = 0; r < nrows; r++) {
        for (int64_t b = 0; b < nb; b++) {
            float v[32];
            for (int i = 0; i < 32; i++) {
                int64_t c = b * 32 + i;
                v[i] = c < ncols ? x[r * ncols + c] : 0.0f;
            }
            q8_1_block(v, out + (r * nb + b) * 36);
        }
    }
}

/* Q8_0 weight quantizer, kv_q8_0.rs:49-89. */
void orc_quantize_q8_0(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float *v = x + b * 32;
        uint8_t *o = out + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) { float a = fabsf(v[i]); if (a > amax) amax = a; }
        float scale = amax / 127.0f;
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        wr16(o, orc_f32_to_f16(scale));
        for (int i = 0; i < 32; i++) {
            float q = roundf(v[i] * inv);
            q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* Q4_0 weight quantizer.  The reference holds no Q4_0 quantizer; this is
 * ggml's published reference rule: m = element of largest magnitude,
 * d = m / -8, q = min(15, trunc(x/d + 8.5)), d stored as f16. */
void orc_quantize_q4_0(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float *v = x + b * 32;
        uint8_t *o = out + b * 18;
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; i++) if (amax < fabsf(v[i])) { amax = fabsf(v[i]); mx = v[i]; }
        float d = mx / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(o, orc_f32_to_f16(d));
        for (int j = 0; j < 16; j++) {
            int a = (int)(v[j] * id + 8.5f), c = (int)(v[j + 16] * id + 8.5f);
            a = a < 0 ? 0 : (a > 15 ? 15 : a);
            c = c < 0 ? 0 : (c > 15 ? 15 : c);
            o[2 + j] = (uint8_t)(a | (c << 4));
        }
    }
}

/* IQ3_S encoder (this build's own; the reference holds none).  Per
 * 256-superblock: d = f16(amax / 465); per 32-sub-block the smallest odd
 * multiplier m = 1+2s with 15*d*m >= sub-amax; per group of 4 the grid
 * entry nearest (squared error, lowest index on ties) to |x| / (d*m);
 * sign bits from x < 0.  Every step is an IEEE operation, so the GPU
 * encoder in the library reproduces it byte for byte. */
void orc_quantize_iq3_s(const float *x, int64_t n, uint8_t *out) {
    for (int64_t sb = 0; sb < n / 256; sb++) {
        const float *v = x + sb * 256;
        uint8_t *o = out + sb * 110;
        memset(o, 0, 110);
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) { float a = fabsf(v[i]); amax = a > amax ? a : amax; }
        uint16_t dh = orc_f32_to_f16(amax / 465.0f);
        float dd = orc_f16_to_f32(dh);
        if (!(dd > 0.0f)) continue;
        wr16(o, dh);
        for (int ib = 0; ib < 8; ib++) {
            const float *w = v + ib * 32;
            float sa = 0.0f;
            for (int i = 0; i < 32; i++) { float a = fabsf(w[i]); sa = a > sa ? a : sa; }
            float t = sa / (15.0f * dd);
            int s = (int)ceilf((t - 1.0f) * 0.5f);
            s = s < 0 ? 0 : (s > 15 ? 15 : s);
            float den = dd * (float)(1 + 2 * s);
            for (int l = 0; l < 4; l++) {
                uint8_t sg = 0;
                for (int h = 0; h < 2; h++) {
                    float lv[4];
                    for (int j = 0; j < 4; j++) {
                        float xv = w[8 * l + 4 * h + j];
                        lv[j] = fabsf(xv) / den;
                        if (xv < 0.0f) sg |= (uint8_t)(1u << (4 * h + j));
                    }
                    int best = 0;
                    float berr = INFINITY;
                    for (int g = 0; g < 512; g++) {
                        uint32_t gv = orc_iq3s_grid[g];
                        float err = 0.0f;
                        for (int j = 0; j < 4; j++) {
                            float df = lv[j] - (float)((gv >> (8 * j)) & 0xFFu);
                            err = fmaf(df, df, err);
                        }
                        if (err < berr) { berr = err; best = g; }
                    }
                    o[2 + 8 * ib + 2 * l + h] = (uint8_t)(best & 0xFF);
                    o[66 + ib] |= (uint8_t)(((best >> 8) & 1) << (2 * l + h));
                }
                o[74 + 4 * ib + l] = sg;
            }
            o[106 + ib / 2] |= (uint8_t)(s << (4 * (ib & 1)));
        }
    }
}

/* signed level of element e (0..31) of IQ3_S sub-block ib, without scales */
static inline int iq3s_level(const uint8_t *blk, int ib, int e) {
    int l = e >> 3, h = (e >> 2) & 1, j = e & 3;
    int qh = blk[66 + ib];
    int idx = blk[2 + 8 * ib + 2 * l + h] | (((qh >> (2 * l + h)) & 1) << 8);
    int g = (int)((orc_iq3s_grid[idx] >> (8 * j)) & 0xFFu);
    return (blk[74 + 4 * ib + l] >> (4 * h + j)) & 1 ? -g : g;
}
static inline int iq3s_mult(const uint8_t *blk, int ib) {
    return 1 + 2 * ((blk[106 + ib / 2] >> (4 * (ib & 1))) & 0xF);
}

/* Q4_K / Q5_K 6-bit scale and min of sub-block j (gguf_loader.rs:1150-1163) */
static void kq_scale_min(const uint8_t *sc12, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = sc12[j] & 63;
        *m = sc12[j + 4] & 63;
    } else {
        *sc = (sc12[j + 4] & 0xF) | ((sc12[j - 4] >> 6) << 4);
        *m = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
    }
}
/* unsigned quant of element e (0..31) of sub-block ib: Q4_K 0..15, Q5_K 0..31 */
static inline int q4k_quant(const uint8_t *blk, int ib, int e) {
    return (blk[16 + 32 * (ib / 2) + e] >> (4 * (ib & 1))) & 0xF;
}
static inline int q5k_quant(const uint8_t *blk, int ib, int e) {
    return ((blk[48 + 32 * (ib / 2) + e] >> (4 * (ib & 1))) & 0xF) | (((blk[16 + e] >> ib) & 1) << 4);
}
/* Q6_K signed quant (q - 32) of element e of sub-block ib, and its int8 scale */
static inline int q6k_quant(const uint8_t *blk, int ib, int e) {
    int gi = ib / 4, jj = ib % 4;
    int lo = (blk[64 * gi + 32 * (jj & 1) + e] >> (4 * (jj >> 1))) & 0xF;
    int hi = (blk[128 + 32 * gi + e] >> (2 * jj)) & 3;
    return (lo | (hi << 4)) - 32;
}
static inline int q6k_scale(const uint8_t *blk, int ib, int e) {
    return (int8_t)blk[192 + 8 * (ib / 4) + 2 * (ib % 4) + e / 16];
}
static const int8_t mxfp4_level[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
static inline float e8m0_half(uint8_t e) {   /* 2^(e-128), exact */
    uint32_t bits = e >= 2 ? (uint32_t)(e - 1) << 23 : 0x00200000u << e;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
static inline int mxfp4_quant(const uint8_t *blk, int e) {
    return mxfp4_level[e < 16 ? blk[1 + e] & 0xF : blk[1 + e - 16] >> 4];
}

void orc_dequantize(int type, const uint8_t *w, int64_t n, float *out) {
    if (type == ORC_Q8_0) {
        for (int64_t b = 0; b < n / 32; b++) {
            float d = orc_f16_to_f32(rd16(w + b * 34));
            for (int i = 0; i < 32; i++) out[b * 32 + i] = (float)(int8_t)w[b * 34 + 2 + i] * d;
        }
    } else if (type == ORC_Q4_0) {
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t *o = w + b * 18;
            float d = orc_f16_to_f32(rd16(o));
            for (int j = 0; j < 16; j++) {
                out[b * 32 + j] = (float)((o[2 + j] & 0xF) - 8) * d;
                out[b * 32 + j + 16] = (float)((o[2 + j] >> 4) - 8) * d;
            }
        }
    } else if (type == ORC_IQ3_S) {
        for (int64_t sb = 0; sb < n / 256; sb++) {
            const uint8_t *o = w + sb * 110;
            float d = orc_f16_to_f32(rd16(o));
            for (int ib = 0; ib < 8; ib++) {
                float db = d * (float)iq3s_mult(o, ib);
                for (int e = 0; e < 32; e++) out[sb * 256 + ib * 32 + e] = db * (float)iq3s_level(o, ib, e);
            }
        }
    } else if (type == ORC_Q4_K || type == ORC_Q5_K) {
        /* gguf_loader.rs:1228-1257 / :1310-1327: d*sc*q - dmin*m */
        const int bytes = type == ORC_Q4_K ? 144 : 176;
        for (int64_t sb = 0; sb < n / 256; sb++) {
            const uint8_t *o = w + sb * bytes;
            float d = orc_f16_to_f32(rd16(o)), dmin = orc_f16_to_f32(rd16(o + 2));
            for (int ib = 0; ib < 8; ib++) {
                int sc, m;
                kq_scale_min(o + 4, ib, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                for (int e = 0; e < 32; e++) {
                    int q = type == ORC_Q4_K ? q4k_quant(o, ib, e) : q5k_quant(o, ib, e);
                    out[sb * 256 + ib * 32 + e] = d1 * (float)q - m1;
                }
            }
        }
    } else if (type == ORC_Q6_K) {
        for (int64_t sb = 0; sb < n / 256; sb++) {
            const uint8_t *o = w + sb * 210;
            float d = orc_f16_to_f32(rd16(o + 208));
            for (int ib = 0; ib < 8; ib++)
                for (int e = 0; e < 32; e++)
                    out[sb * 256 + ib * 32 + e] = d * (float)q6k_scale(o, ib, e) * (float)q6k_quant(o, ib, e);
        }
    } else if (type == ORC_MXFP4) {
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t *o = w + b * 17;
            float d = e8m0_half(o[0]);
            for (int e = 0; e < 32; e++) out[b * 32 + e] = (float)mxfp4_quant(o, e) * d;
        }
    }
}

/* ---------------------------------------------------------- block dots */

/* int32 dot of weight block b of a row with the Q8_1 block b; *scale gets
 * f32(d_w) * f32(d_x).  Q4_K / Q5_K also give the min term's integer
 * m * sum(q_x) in *s2 and its scale -(f32(dmin) * f32(d_x)) in *scale2
 * (*s2 = 0 for the other types). */
static inline int32_t block_dot2(int type, const uint8_t *row, const uint8_t *xq, int b, float *scale,
                                 int32_t *s2, float *scale2) {
    const uint8_t *xb = xq + (int64_t)b * 36;
    const int8_t *qx = (const int8_t *)(xb + 4);
    float dx = orc_f16_to_f32(rd16(xb));
    int32_t s = 0;
    *s2 = 0;
    *scale2 = 0.0f;
    if (type == ORC_Q8_0) {
        const uint8_t *o = row + (int64_t)b * 34;
        for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)o[2 + i] * qx[i];
        *scale = orc_f16_to_f32(rd16(o)) * dx;
    } else if (type == ORC_Q4_0) {
        const uint8_t *o = row + (int64_t)b * 18;
        for (int j = 0; j < 16; j++) {
            s += ((o[2 + j] & 0xF) - 8) * qx[j];
            s += ((o[2 + j] >> 4) - 8) * qx[j + 16];
        }
        *scale = orc_f16_to_f32(rd16(o)) * dx;
    } else if (type == ORC_Q4_0_SFORM) {
        /* unsigned nibbles; the caller forms ggml's term (row_dot) */
        const uint8_t *o = row + (int64_t)b * 18;
        for (int j = 0; j < 16; j++) {
            s += (o[2 + j] & 0xF) * qx[j];
            s += (o[2 + j] >> 4) * qx[j + 16];
        }
        *scale = orc_f16_to_f32(rd16(o));                    /* d_w */
        *scale2 = -(8.0f * orc_f16_to_f32(rd16(xb + 2)));   /* -8 s_x */
    } else if (type == ORC_IQ3_S) {
        const uint8_t *o = row + (int64_t)(b >> 3) * 110;
        int ib = b & 7;
        for (int e = 0; e < 32; e++) s += iq3s_level(o, ib, e) * qx[e];
        s *= iq3s_mult(o, ib);
        *scale = orc_f16_to_f32(rd16(o)) * dx;
    } else if (type == ORC_Q4_K || type == ORC_Q5_K) {
        const uint8_t *o = row + (int64_t)(b >> 3) * (type == ORC_Q4_K ? 144 : 176);
        int ib = b & 7, sc, m, sx = 0;
        kq_scale_min(o + 4, ib, &sc, &m);
        for (int e = 0; e < 32; e++) {
            s += (type == ORC_Q4_K ? q4k_quant(o, ib, e) : q5k_quant(o, ib, e)) * qx[e];
            sx += qx[e];
        }
        s *= sc;
        *scale = orc_f16_to_f32(rd16(o)) * dx;
        *s2 = m * sx;
        *scale2 = -(orc_f16_to_f32(rd16(o + 2)) * dx);
    } else if (type == ORC_Q6_K) {
        const uint8_t *o = row + (int64_t)(b >> 3) * 210;
        int ib = b & 7, lo = 0, hi = 0;
        for (int e = 0; e < 16; e++) lo += q6k_quant(o, ib, e) * qx[e];
        for (int e = 16; e < 32; e++) hi += q6k_quant(o, ib, e) * qx[e];
        s = q6k_scale(o, ib, 0) * lo + q6k_scale(o, ib, 16) * hi;
        *scale = orc_f16_to_f32(rd16(o + 208)) * dx;
    } else if (type == ORC_MXFP4) {
        const uint8_t *o = row + (int64_t)b * 17;
        for (int e = 0; e < 32; e++) s += mxfp4_quant(o, e) * qx[e];
        *scale = e8m0_half(o[0]) * dx;
    }
    return s;
}
static inline int32_t block_dot(int type, const uint8_t *row, const uint8_t *xq, int b, float *scale) {
    int32_t s2;
    float sc2;
    return block_dot2(type, row, xq, b, scale, &s2, &sc2);
}

void orc_block_dots(int type, const uint8_t *W, const uint8_t *xq,
                    int ncols, int nrows, int32_t *out) {
    int nb = ncols / 32;
    int64_t rb = orc_row_bytes(type, ncols);
    for (int r = 0; r < nrows; r++) {
        float sc;
        for (int b = 0; b < nb; b++) out[(int64_t)r * nb + b] = block_dot(type, W + r * rb, xq, b, &sc);
    }
}

static float row_dot(int type, const uint8_t *row, const uint8_t *xq, int nb, int L, int G) {
    float acc[256];
    for (int j = 0; j < L; j++) acc[j] = 0.0f;
    for (int b = 0; b < nb; b++) {
        float sc, sc2;
        int32_t s2;
        int32_t s = block_dot2(type, row, xq, b, &sc, &s2, &sc2);
        int j = (b / G) % L;
        if (type == ORC_Q4_0_SFORM) {
            /* ggml mul_mat_vec_q4_0_q8_1's block term (out of tree; the
             * contraction nvcc's default fmad gives it) */
            const float dx = orc_f16_to_f32(rd16(xq + (int64_t)b * 36));
            acc[j] = fmaf(sc, fmaf((float)s, dx, sc2), acc[j]);
            continue;
        }
        acc[j] = fmaf(sc, (float)s, acc[j]);
        if (type == ORC_Q4_K || type == ORC_Q5_K) acc[j] = fmaf(sc2, (float)s2, acc[j]);
    }
    for (int m = L / 2; m >= 1; m >>= 1)
        for (int i = 0; i < m; i++) acc[i] = acc[i] + acc[i + m];
    return acc[0];
}

void orc_gemv(int type, const uint8_t *W, const uint8_t *xq, int64_t xq_stride,
              float *y, int ncols, int nrows, int ntok, int L, int G, int nthreads) {
    int nb = ncols / 32;
    int64_t rb = orc_row_bytes(type, ncols);
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
    for (int r = 0; r < nrows; r++)
        for (int t = 0; t < ntok; t++)
            y[(int64_t)t * nrows + r] = row_dot(type, W + (int64_t)r * rb, xq + t * xq_stride, nb, L, G);
    (void)nthreads;
}

void orc_gemv_q8_0_f64(const uint8_t *W, const float *x, float *y, int ncols, int nrows) {
    int nb = ncols / 32;
    for (int r = 0; r < nrows; r++) {
        double sum = 0.0;
        for (int b = 0; b < nb; b++) {
            const uint8_t *o = W + ((int64_t)r * nb + b) * 34;
            double sc = (double)orc_f16_to_f32(rd16(o));
            for (int i = 0; i < 32; i++) sum += sc * (double)(int8_t)o[2 + i] * (double)x[b * 32 + i];
        }
        y[r] = (float)sum;
    }
}

/* ------------------------------------------------------------- routing */

/* 256 strided slots with fused multiply-add, then a halving tree
 * (elementwise.rs:186-221 launched with 256 threads). */
static float dot256(const float *a, const float *x, int H) {
    float acc[256];
    for (int t = 0; t < 256; t++) acc[t] = 0.0f;
    for (int j = 0; j < H; j++) acc[j & 255] = fmaf(a[j], x[j], acc[j & 255]);
    for (int m = 128; m >= 1; m >>= 1)
        for (int i = 0; i < m; i++) acc[i] = acc[i] + acc[i + m];
    return acc[0];
}

void orc_router(const float *Wr, const float *x, float *logits, int E, int H) {
    for (int e = 0; e < E; e++) logits[e] = dot256(Wr + (int64_t)e * H, x, H);
}

void orc_topk_softmax(const float *logits, int E, int K, int32_t *idx, float *w) {
    float p[1024], ev[1024];
    float mx = logits[0];
    for (int i = 1; i < E; i++) mx = fmaxf(mx, logits[i]);
    for (int i = 0; i < E; i++) { ev[i] = orc_exp(logits[i] - mx); p[i] = ev[i]; }
    for (int st = 512; st >= 1; st >>= 1)
        for (int t = 0; t < st; t++)
            if (t + st < E) p[t] += p[t + st];
    float sum = p[0];
    for (int i = 0; i < E; i++) p[i] = sum > 0.0f ? ev[i] / sum : 1.0f / (float)E;
    float wsum = 0.0f;
    for (int k = 0; k < K; k++) {
        int bi = 0;
        float bv = -1.0f;
        for (int i = 0; i < E; i++) if (p[i] > bv) { bv = p[i]; bi = i; }
        idx[k] = bi;
        w[k] = bv;
        wsum += bv;
        p[bi] = -1.0f;
    }
    if (wsum > 0.0f) {
        float inv = 1.0f / wsum;
        for (int k = 0; k < K; k++) w[k] *= inv;
    }
}

/* ------------------------------------------------------------------ MoE */

static int64_t pad512(int64_t n) { return (n + 511) / 512 * 512; }

static void expert_ffn(int type, const uint8_t *g, const uint8_t *u, const uint8_t *dn,
                       const uint8_t *xq, int H, int F, int L, int G, float *out, int nthreads) {
    float *gv = malloc(sizeof(float) * F), *uv = malloc(sizeof(float) * F), *h = malloc(sizeof(float) * F);
    uint8_t *hq = malloc(pad512(F) / 32 * 36);
    orc_gemv(type, g, xq, 0, gv, H, F, 1, L, G, nthreads);
    orc_gemv(type, u, xq, 0, uv, H, F, 1, L, G, nthreads);
    for (int i = 0; i < F; i++) h[i] = orc_silu(gv[i]) * uv[i];
    orc_quantize_q8_1(h, F, pad512(F), 1, hq);
    orc_gemv(type, dn, hq, 0, out, F, H, 1, L, G, nthreads);
    free(gv); free(uv); free(h); free(hq);
}

void orc_moe(const orc_moe_params *p, const float *x, float *out,
             int32_t *ids, float *wts, int nthreads) {
    int H = p->H, F = p->F, E = p->E, K = p->K;
    float *logits = malloc(sizeof(float) * E);
    float *dn = malloc(sizeof(float) * H);
    float *acc = malloc(sizeof(float) * H);
    uint8_t *xq = malloc(pad512(H) / 32 * 36);
    int32_t id[1024];
    float w[1024];
    for (int t = 0; t < p->M; t++) {
        const float *xt = x + (int64_t)t * H;
        orc_router(p->router, xt, logits, E, H);
        if (p->logit_bias) for (int e = 0; e < E; e++) logits[e] = logits[e] + p->logit_bias[e];
        orc_topk_softmax(logits, E, K, id, w);
        if (ids) memcpy(ids + (int64_t)t * K, id, sizeof(int32_t) * K);
        if (wts) memcpy(wts + (int64_t)t * K, w, sizeof(float) * K);
        orc_quantize_q8_1(xt, H, pad512(H), 1, xq);
        for (int i = 0; i < H; i++) acc[i] = 0.0f;
        for (int k = 0; k < K; k++) {
            int e = id[k];
            expert_ffn(p->exp_type, p->gate + e * p->stride_gate, p->up + e * p->stride_up,
                       p->down + e * p->stride_down, xq, H, F, p->L, p->G, dn, nthreads);
            for (int i = 0; i < H; i++) acc[i] = fmaf(w[k], dn[i], acc[i]);
        }
        float *o = out + (int64_t)t * H;
        if (p->sh_type >= 0) {
            expert_ffn(p->sh_type, p->sh_gate, p->sh_up, p->sh_down, xq, H, F, p->L, p->G, dn, nthreads);
            if (p->sh_gate_w) {
                float gl = dot256(p->sh_gate_w, xt, H);
                float sc = 1.0f / (1.0f + orc_exp(-gl));
                for (int i = 0; i < H; i++) o[i] = fmaf(dn[i], sc, acc[i]);
            } else {
                for (int i = 0; i < H; i++) o[i] = dn[i] + acc[i];
            }
        } else {
            memcpy(o, acc, sizeof(float) * H);
        }
    }
    free(logits); free(dn); free(acc); free(xq);
}

/* ------------------------------------------- fused MoE on f32 activations
 * The reference's fused_moe_iq3s (cs/src/kernels/fused_moe.rs:101-311 =
 * cs/kernels/chimere_kernels.cu:1093-1143): per selected expert, gate / up
 * rows of IQ3_S weights against f32 x, h = silu(g) * u, down rows against h,
 * output += w_k * y_k.  The reference sums each row sequentially in one
 * thread (fma of d * (1 + 2 sc) * level * sign with x) and adds the experts'
 * terms by atomicAdd, in no fixed order; restated here in the HIP kernels'
 * fixed order (chimere_amd/csrc/fused_moe.hip): lane j = b % L of a row
 * (gate / up rows L = 64, down rows L = 16) takes its 32-element blocks in
 * ascending order, a block's s = fmaf(level_e, x_e, s) over e = 0..31,
 * acc_j = fmaf(f32(d) * (1 + 2 sc), s, acc_j), lanes by the halving tree;
 * output[r] = output[r] + a, a = fmaf(w_k, y_k[r], a) for k ascending. */
static float iq3s_row_f32(const uint8_t *row, const float *x, int nb, int L) {
    float acc[64];
    for (int j = 0; j < L; j++) acc[j] = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (int64_t)(b >> 3) * 110;
        const int ib = b & 7;
        float s = 0.0f;
        for (int e = 0; e < 32; e++) s = fmaf((float)iq3s_level(blk, ib, e), x[32 * b + e], s);
        const float scale = orc_f16_to_f32(rd16(blk)) * (float)iq3s_mult(blk, ib);
        acc[b % L] = fmaf(scale, s, acc[b % L]);
    }
    for (int m = L / 2; m >= 1; m >>= 1)
        for (int i = 0; i < m; i++) acc[i] = acc[i] + acc[i + m];
    return acc[0];
}

void orc_fused_moe_iq3s(const float *x, const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                        const int32_t *ids, const float *wts, float *out, int H, int F,
                        int64_t bg, int64_t bu, int64_t bd, int K) {
    const int64_t rbH = (int64_t)H / 256 * 110, rbF = (int64_t)F / 256 * 110;
    float *h = malloc(sizeof(float) * (size_t)K * F);
    for (int k = 0; k < K; k++)
        for (int f = 0; f < F; f++) {
            const float g = iq3s_row_f32(gate + ids[k] * bg + f * rbH, x, H / 32, 64);
            const float u = iq3s_row_f32(up + ids[k] * bu + f * rbH, x, H / 32, 64);
            h[(int64_t)k * F + f] = orc_silu(g) * u;
        }
    for (int r = 0; r < H; r++) {
        float a = 0.0f;
        for (int k = 0; k < K; k++)
            a = fmaf(wts[k], iq3s_row_f32(down + ids[k] * bd + r * rbF, h + (int64_t)k * F, F / 32, 16), a);
        out[r] = out[r] + a;
    }
    free(h);
}

/* ------------------------------------------------------------ ncmoe path
 * The reference's CPU expert path (cs/src/qwen35_model/moe_ffn.rs:1507-1591)
 * over its ggml wrapper (cs/ffi/ggml_iq3s_gemv.c:33-127): activations to
 * Q8_K once per GEMV, one IQ3_S x Q8_K dot per row.  ggml itself (ik_llama.cpp)
 * is out of tree; its published semantics are restated here.
 *
 * Q8_K block, 296 B (layout cs/ffi/ggml_iq3s_gemv.h:14-16): f32 d, f32 sum,
 * int8 qs[256], int16 bsums[16].  quantize_row_q8_K: max = the element of
 * largest |x| (the first one); amax == 0 -> all fields zero; otherwise
 * iscale = -127 / max, q = min(127, round-half-even(iscale * x)), bsums =
 * sums of 16 quants, d = 1 / iscale; sum = d * sum(q) (a field the IQ3_S dot
 * does not read). */
void orc_quantize_q8_K(const float *x, int64_t k, uint8_t *out) {
    for (int64_t b = 0; b < k / 256; b++) {
        const float *v = x + b * 256;
        uint8_t *o = out + b * 296;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 256; j++) {
            float ax = fabsf(v[j]);
            if (ax > amax) { amax = ax; max = v[j]; }
        }
        memset(o, 0, 296);
        if (amax == 0.0f) continue;
        const float iscale = -127.0f / max;
        int8_t *q = (int8_t *)(o + 8);
        int sq = 0;
        for (int j = 0; j < 256; j++) {
            int t = (int)rintf(iscale * v[j]);
            q[j] = (int8_t)(t < 127 ? t : 127);
            sq += q[j];
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) s += q[16 * g + j];
            int16_t s16 = (int16_t)s;
            memcpy(o + 264 + 2 * g, &s16, 2);
        }
        const float d = 1.0f / iscale, sum = d * (float)sq;
        memcpy(o, &d, 4);
        memcpy(o + 4, &sum, 4);
    }
}

/* IQ3_S super-block(s) x Q8_K: per super-block the exact integer
 * bsum = sum_ib (1 + 2 s_ib) * sum_e level_e * q_e, then, in super-block
 * order, acc = fmaf(f32(d_w) * d_y, (float)bsum, acc) (ggml's generic
 * `sumf += d * bsum` as contracted). */
float orc_vec_dot_iq3s_q8K(int n, const uint8_t *w, const uint8_t *y) {
    float acc = 0.0f;
    for (int b = 0; b < n / 256; b++) {
        const uint8_t *o = w + (int64_t)b * 110, *yb = y + (int64_t)b * 296;
        const int8_t *q = (const int8_t *)(yb + 8);
        float dy;
        memcpy(&dy, yb, 4);
        int32_t bsum = 0;
        for (int ib = 0; ib < 8; ib++) {
            int32_t s = 0;
            for (int e = 0; e < 32; e++) s += iq3s_level(o, ib, e) * q[32 * ib + e];
            bsum += s * iq3s_mult(o, ib);
        }
        acc = fmaf(orc_f16_to_f32(rd16(o)) * dy, (float)bsum, acc);
    }
    return acc;
}

void orc_gemv_iq3s_q8K(const uint8_t *W, const float *x, float *y, int nrows, int ncols) {
    uint8_t *xq = (uint8_t *)malloc((size_t)(ncols / 256) * 296);
    orc_quantize_q8_K(x, ncols, xq);
    const int64_t rb = (int64_t)ncols / 256 * 110;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int r = 0; r < nrows; r++) y[r] = orc_vec_dot_iq3s_q8K(ncols, W + r * rb, xq);
    free(xq);
}

/* The expert loop of one token (moe_ffn.rs:1538-1585): for each selected
 * (expert, weight) in order: gate = W_g x and up = W_u x (IQ3_S x Q8_K),
 * h = silu(gate) * up in f32 with expf (g / (1 + exp(-g)), as the Rust
 * code), down = W_d h, combined += weight * down (a product then a sum). */
void orc_ncmoe(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int64_t sg, int64_t su, int64_t sd,
               const int32_t *ids, const float *wts, int K, const float *x, float *out, int H, int F) {
    float *g = (float *)malloc(sizeof(float) * (size_t)F), *u = (float *)malloc(sizeof(float) * (size_t)F);
    float *dn = (float *)malloc(sizeof(float) * (size_t)H);
    for (int i = 0; i < H; i++) out[i] = 0.0f;
    for (int k = 0; k < K; k++) {
        const int64_t e = ids[k];
        orc_gemv_iq3s_q8K(gate + e * sg, x, g, F, H);
        orc_gemv_iq3s_q8K(up + e * su, x, u, F, H);
        for (int i = 0; i < F; i++) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        orc_gemv_iq3s_q8K(down + e * sd, g, dn, H, F);
        for (int i = 0; i < H; i++) out[i] = out[i] + wts[k] * dn[i];
    }
    free(g); free(u); free(dn);
}

/* One MoE layer with the routed experts on the CPU path (moe_ffn.rs:1507-1591)
 * and everything else as orc_moe: router, top-k, then the shared expert on
 * the Q8_1 path combined with the CPU experts' sum.  IQ3_S experts only. */
void orc_moe_ncmoe(const orc_moe_params *p, const float *x, float *out, int32_t *ids, float *wts, int nthreads) {
    int H = p->H, F = p->F, E = p->E, K = p->K;
    float *logits = malloc(sizeof(float) * E);
    float *dn = malloc(sizeof(float) * H);
    float *acc = malloc(sizeof(float) * H);
    uint8_t *xq = malloc(pad512(H) / 32 * 36);
    int32_t id[1024];
    float w[1024];
    for (int t = 0; t < p->M; t++) {
        const float *xt = x + (int64_t)t * H;
        orc_router(p->router, xt, logits, E, H);
        if (p->logit_bias) for (int e = 0; e < E; e++) logits[e] = logits[e] + p->logit_bias[e];
        orc_topk_softmax(logits, E, K, id, w);
        if (ids) memcpy(ids + (int64_t)t * K, id, sizeof(int32_t) * K);
        if (wts) memcpy(wts + (int64_t)t * K, w, sizeof(float) * K);
        orc_ncmoe(p->gate, p->up, p->down, p->stride_gate, p->stride_up, p->stride_down, id, w, K, xt, acc, H, F);
        float *o = out + (int64_t)t * H;
        if (p->sh_type >= 0) {
            orc_quantize_q8_1(xt, H, pad512(H), 1, xq);
            expert_ffn(p->sh_type, p->sh_gate, p->sh_up, p->sh_down, xq, H, F, p->L, p->G, dn, nthreads);
            if (p->sh_gate_w) {
                float gl = dot256(p->sh_gate_w, xt, H);
                float sc = 1.0f / (1.0f + orc_exp(-gl));
                for (int i = 0; i < H; i++) o[i] = fmaf(dn[i], sc, acc[i]);
            } else {
                for (int i = 0; i < H; i++) o[i] = dn[i] + acc[i];
            }
        } else {
            memcpy(o, acc, sizeof(float) * H);
        }
    }
    free(logits); free(dn); free(acc); free(xq);
}
