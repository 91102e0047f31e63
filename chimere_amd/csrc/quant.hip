// quant.hip -- Q8_1 activation quantizer and device weight quantizers.
#include "api_internal.h"
#include "common.h"

namespace chimere {

// Q8_1 with ggml semantics (cs/kernels/chimere_kernels.cu:1495-1523): one
// 32-lane half-wave per block; amax and sum reduced with xor masks
// 16,8,4,2,1 confined to the 32 lanes; d = amax/127 (IEEE division),
// q = amax==0 ? 0 : roundf(x/d) (half away from zero), ds = (f16(d), f16(sum)).
// Grid: x over groups of 8 blocks of one row, y over rows.
__global__ __launch_bounds__(256) void k_quantize_q8_1(const float* __restrict__ x,
                                                       uint8_t* __restrict__ out, int64_t ncols,
                                                       int64_t ncols_padded) {
    const int64_t row = blockIdx.y;
    const int64_t nb = ncols_padded / QK;
    const int64_t b = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int i = threadIdx.x & 31;
    if (b >= nb) return;   // whole half-wave exits together
    const int64_t col = b * QK + i;
    float xi = col < ncols ? x[row * ncols + col] : 0.0f;
    const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
    const float d = amax / 127.0f;
    const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
    uint8_t* blk = out + (row * nb + b) * Q8_1_BYTES;
    blk[4 + i] = (uint8_t)(int8_t)q;
    if (i == 0) *(uint32_t*)blk = f2h(d) | (f2h(sum) << 16);
}

void launch_quantize_q8_1(const float* x, void* out, int64_t ncols, int64_t ncols_padded,
                          int64_t nrows, hipStream_t s) {
    dim3 grid((unsigned)((ncols_padded / QK + 7) / 8), (unsigned)nrows);
    hipLaunchKernelGGL(k_quantize_q8_1, grid, dim3(256), 0, s, x, (uint8_t*)out, ncols,
                       ncols_padded);
}

// ---- weight quantizers (one thread per 32-block / per 64-element IQ3_S pair)

__global__ void k_quant_q8_0(const float* __restrict__ x, uint8_t* __restrict__ out, int64_t nb) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* v = x + b * 32;
    uint8_t* o = out + b * 34;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { float a = __builtin_fabsf(v[i]); if (a > amax) amax = a; }
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    uint32_t h = f2h(scale);
    o[0] = (uint8_t)h; o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) {
        float q = __builtin_roundf(v[i] * inv);
        q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
        o[2 + i] = (uint8_t)(int8_t)q;
    }
}

__global__ void k_quant_q4_0(const float* __restrict__ x, uint8_t* __restrict__ out, int64_t nb) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* v = x + b * 32;
    uint8_t* o = out + b * 18;
    float amax = 0.0f, mx = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = __builtin_fabsf(v[i]);
        if (amax < a) { amax = a; mx = v[i]; }
    }
    float d = mx / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    // an all-zero block has d = 0 / -8 = -0.0 (f16 0x8000), as the reference
    // rule produces; spelled out because the compiler may fold the sign away
    uint32_t h = mx == 0.0f ? 0x8000u : f2h(d);
    o[0] = (uint8_t)h; o[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 16; j++) {
        int a = (int)(v[j] * id + 8.5f), c = (int)(v[j + 16] * id + 8.5f);
        a = a < 0 ? 0 : (a > 15 ? 15 : a);
        c = c < 0 ? 0 : (c > 15 ? 15 : c);
        o[2 + j] = (uint8_t)(a | (c << 4));
    }
}

__constant__ uint32_t c_iq3s_grid[512] = CHIMERE_IQ3S_GRID_INIT;

// IQ3_S encoder: per 256-superblock d = f16(amax/465); per sub-block the
// smallest odd multiplier m = 1+2s with 15*d*m >= sub-amax; per group of 4
// values the codebook entry nearest (squared error, lowest index on ties) to
// |x|/(d*m); sign bits from x < 0.  One thread per pair of sub-blocks (so it
// owns a whole scale byte); the codebook is staged in LDS.
__global__ __launch_bounds__(256) void k_quant_iq3_s(const float* __restrict__ x,
                                                     uint8_t* __restrict__ out, int64_t nsb) {
    __shared__ uint32_t grid[512];
    for (int i = threadIdx.x; i < 512; i += blockDim.x) grid[i] = c_iq3s_grid[i];
    __syncthreads();
    int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nsb * 4) return;
    const int64_t sb = p >> 2;
    const int pair = (int)(p & 3);
    const float* v = x + sb * 256;
    uint8_t* o = out + sb * 110;
    float amax = 0.0f;
    for (int i = 0; i < 256; i++) { float a = __builtin_fabsf(v[i]); amax = a > amax ? a : amax; }
    uint32_t dh = f2h(amax / 465.0f);
    float dd = h2f(dh);
    const bool zero = !(dd > 0.0f);
    if (pair == 0) { o[0] = zero ? 0 : (uint8_t)dh; o[1] = zero ? 0 : (uint8_t)(dh >> 8); }
    uint8_t scale_byte = 0;
    for (int h2 = 0; h2 < 2; h2++) {
        const int ib = pair * 2 + h2;
        const float* w = v + ib * 32;
        uint8_t qh = 0;
        if (zero) {
            for (int i = 0; i < 8; i++) o[2 + 8 * ib + i] = 0;
            for (int l = 0; l < 4; l++) o[74 + 4 * ib + l] = 0;
            o[66 + ib] = 0;
            continue;
        }
        float sa = 0.0f;
        for (int i = 0; i < 32; i++) { float a = __builtin_fabsf(w[i]); sa = a > sa ? a : sa; }
        float t = sa / (15.0f * dd);
        int s = (int)__builtin_ceilf((t - 1.0f) * 0.5f);
        s = s < 0 ? 0 : (s > 15 ? 15 : s);
        float den = dd * (float)(1 + 2 * s);
        for (int l = 0; l < 4; l++) {
            uint8_t sg = 0;
            for (int h = 0; h < 2; h++) {
                float lv[4];
                for (int j = 0; j < 4; j++) {
                    float xv = w[8 * l + 4 * h + j];
                    lv[j] = __builtin_fabsf(xv) / den;
                    if (xv < 0.0f) sg |= (uint8_t)(1u << (4 * h + j));
                }
                int best = 0;
                float berr = __builtin_huge_valf();
                for (int g = 0; g < 512; g++) {
                    uint32_t gv = grid[g];
                    float err = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float df = lv[j] - (float)((gv >> (8 * j)) & 0xFFu);
                        err = __builtin_fmaf(df, df, err);
                    }
                    if (err < berr) { berr = err; best = g; }
                }
                o[2 + 8 * ib + 2 * l + h] = (uint8_t)(best & 0xFF);
                qh |= (uint8_t)(((best >> 8) & 1) << (2 * l + h));
            }
            o[74 + 4 * ib + l] = sg;
        }
        o[66 + ib] = qh;
        scale_byte |= (uint8_t)(s << (4 * h2));
    }
    o[106 + pair] = scale_byte;
}

}  // namespace chimere

using namespace chimere;

extern "C" {

void chimere_quantize_q8_1(const float* input, void* output, int64_t ncols, int64_t ncols_padded,
                           hipStream_t stream) {
    chimere_quantize_q8_1_batched(input, output, ncols, ncols_padded, 1, stream);
}

void chimere_quantize_q8_1_batched(const float* input, void* output, int64_t ncols,
                                   int64_t ncols_padded, int batch, hipStream_t stream) {
    CHIMERE_REQUIRE(input && output, CHIMERE_ERR_ARG, "quantize_q8_1: null pointer");
    CHIMERE_REQUIRE(ncols > 0 && ncols_padded >= ncols && ncols_padded % 32 == 0 && batch > 0,
                    CHIMERE_ERR_ARG, "quantize_q8_1: bad sizes ncols=%lld padded=%lld batch=%d",
                    (long long)ncols, (long long)ncols_padded, batch);
    CHIMERE_REQUIRE(((uintptr_t)output & 3) == 0, CHIMERE_ERR_ARG,
                    "quantize_q8_1: output must be 4-byte aligned");
    launch_quantize_q8_1(input, output, ncols, ncols_padded, batch, stream);
    check_launch("quantize_q8_1");
}

void chimere_quantize_weights(int type, const float* x, void* out, int64_t n, hipStream_t stream) {
    CHIMERE_REQUIRE(x && out, CHIMERE_ERR_ARG, "quantize_weights: null pointer");
    if (type == T_Q8_0 || type == T_Q4_0) {
        CHIMERE_REQUIRE(n > 0 && n % 32 == 0, CHIMERE_ERR_ARG, "quantize_weights: n %% 32 != 0");
        int64_t nb = n / 32;
        dim3 grid((unsigned)((nb + 255) / 256));
        if (type == T_Q8_0)
            hipLaunchKernelGGL(k_quant_q8_0, grid, dim3(256), 0, stream, x, (uint8_t*)out, nb);
        else
            hipLaunchKernelGGL(k_quant_q4_0, grid, dim3(256), 0, stream, x, (uint8_t*)out, nb);
    } else if (type == T_IQ3_S) {
        CHIMERE_REQUIRE(n > 0 && n % 256 == 0, CHIMERE_ERR_ARG, "quantize_weights: n %% 256 != 0");
        int64_t nsb = n / 256;
        dim3 grid((unsigned)((nsb * 4 + 255) / 256));
        hipLaunchKernelGGL(k_quant_iq3_s, grid, dim3(256), 0, stream, x, (uint8_t*)out, nsb);
    } else {
        set_error(CHIMERE_ERR_ARG, "quantize_weights: unsupported type %d", type);
        return;
    }
    check_launch("quantize_weights");
}

}  // extern "C"
