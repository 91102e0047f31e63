// moe_common.h -- device helpers shared by the MoE decode and prefill kernels:
// reference-order f32 row dots, softmax/top-k, Q8_1 quantization of blocks.
#pragma once
#include "common.h"

namespace chimere {

constexpr int MAX_TOK = 8;
constexpr int MAX_K = 16;
constexpr int MAX_E = 1024;

// ------------------------------------------------------------ reductions

// Halving-tree sum over 256 threads (stride 128, 64 through LDS, then 32..1
// inside wave 0 by xor shuffles, which equal the halving tree at lane 0).
// Same association as the reference's shared-memory tree
// (elementwise.rs:186-221).  Result valid in thread 0.
__device__ __forceinline__ float tree_sum256(float v, float* red) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    if (tid < 128) red[tid] = red[tid] + red[tid + 128];
    __syncthreads();
    if (tid < 64) {
        float w = red[tid] + red[tid + 64];
        w = w + xlane<32>(w);
        v = bfly32_sum(w);
    }
    __syncthreads();
    return v;
}

// f32 row dot of `a` (H) against NT tokens of x (token stride H), in the
// reference's order: thread t accumulates columns t, t+256, ... with fused
// multiply-add, then tree_sum256.  Results valid in thread 0.
template <int NT>
__device__ __forceinline__ void f32_row_dot(const float* __restrict__ a, const float* __restrict__ x,
                                            int H, int ntok, float* red, float (&out)[NT]) {
    constexpr int U = 8;   // columns per thread loaded together before use
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
    for (int j0 = threadIdx.x; j0 < H; j0 += 256 * U) {
        float av[U];
#pragma unroll
        for (int u = 0; u < U; u++) av[u] = j0 + 256 * u < H ? a[j0 + 256 * u] : 0.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < ntok) {
                float xv[U];
#pragma unroll
                for (int u = 0; u < U; u++) xv[u] = j0 + 256 * u < H ? x[(int64_t)t * H + j0 + 256 * u] : 0.0f;
#pragma unroll
                for (int u = 0; u < U; u++)
                    if (j0 + 256 * u < H) acc[t] = __builtin_fmaf(av[u], xv[u], acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
        if (t < ntok) out[t] = tree_sum256(acc[t], red);
}

// ---------------------------------------------------------------- top-k

// Softmax + top-k + renormalisation of one logits row by ONE wavefront, in
// registers (cs/kernels/chimere_kernels.cu:1150-1223): lane l holds logits
// l, l+64, ... (NV = ceil(E/64) values, zero-padded).  p = exp(l - max) / sum
// where the sum follows the reference's strided halving tree (strides
// 512..64 pair values inside a lane, strides 32..1 pair lanes; padding adds
// +0, which leaves the non-negative partial sums unchanged).
// Selection: the reference takes k rounds of arg-max by probability with ties
// to the lowest index, i.e. the K largest keys (p, -index).  Here the K-th
// largest key is found by a radix select over 41-bit keys
// (f32 bits of p << 11 | 1024 - index) with ballot counts, then each selected
// entry's rank is the number of larger keys -- same set, same order, no
// cross-lane shuffles in the loop.  Weights are renormalised by the
// sequential sum of the selected probabilities (rank order).  Lane k < K
// writes entry k.  Requires E <= 1024, K <= E.
template <int NV>
__device__ __forceinline__ void topk_wave(const float* __restrict__ logits, int E, int K,
                                          int* __restrict__ idx_out, float* __restrict__ w_out) {
    const int lane = threadIdx.x & 63;
    float p[NV], ev[NV];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = lane + 64 * i;
        p[i] = j < E ? logits[j] : -__builtin_huge_valf();
        mx = __builtin_fmaxf(mx, p[i]);
    }
    mx = bfly32_max(__builtin_fmaxf(mx, xlane<32>(mx)));
#pragma unroll
    for (int i = 0; i < NV; i++) {
        ev[i] = (lane + 64 * i) < E ? det_exp(p[i] - mx) : 0.0f;
        p[i] = ev[i];
    }
#pragma unroll
    for (int h = NV / 2; h >= 1; h >>= 1)        // strides 64*h: in-lane pairs
#pragma unroll
        for (int i = 0; i < h; i++) p[i] = p[i] + p[i + h];
    float s = p[0];
    s = bfly32_sum(s + xlane<32>(s));
    // s equals lane 0's value of the halving tree on every lane
    uint64_t key[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = lane + 64 * i;
        p[i] = s > 0.0f ? ev[i] / s : 1.0f / (float)E;
        key[i] = j < E ? (((uint64_t)__builtin_bit_cast(uint32_t, p[i])) << 11) | (uint64_t)(1024 - j) : 0;
    }
    // radix select of the K-th largest key (p <= 1, so the f32 bits fit in 30 bits)
    // (stops as soon as exactly K keys reach the candidate: the set is fixed then)
    uint64_t T = 0;
    for (int b = 40; b >= 0; b--) {
        const uint64_t cand = T | (1ull << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NV; i++) cnt += __popcll(__ballot(key[i] >= cand));
        if (cnt >= K) T = cand;
        if (cnt == K) break;
    }
    // rank each selected entry: rank = number of keys larger than it
    int my_idx = 0;
    float my_w = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        uint64_t m = __ballot(key[i] >= T);
        while (m) {
            const int src = __builtin_ctzll(m);
            m &= m - 1;
            const uint32_t klo = __builtin_amdgcn_readlane((uint32_t)key[i], src);
            const uint32_t khi = __builtin_amdgcn_readlane((uint32_t)(key[i] >> 32), src);
            const uint64_t kx = ((uint64_t)khi << 32) | klo;
            const float px = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[i]), src));
            int r = 0;
#pragma unroll
            for (int i2 = 0; i2 < NV; i2++) r += __popcll(__ballot(key[i2] > kx));
            if (lane == r) { my_idx = src + 64 * i; my_w = px; }
        }
    }
    float ws = 0.0f;
    for (int k = 0; k < K; k++)
        ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), k));
    if (lane < K) {
        idx_out[lane] = my_idx;
        w_out[lane] = ws > 0.0f ? my_w * (1.0f / ws) : my_w;
    }
}

__device__ __forceinline__ void topk_wave_any(const float* logits, int E, int K, int* idx, float* w) {
    if (E <= 64) topk_wave<1>(logits, E, K, idx, w);
    else if (E <= 128) topk_wave<2>(logits, E, K, idx, w);
    else if (E <= 256) topk_wave<4>(logits, E, K, idx, w);
    else if (E <= 512) topk_wave<8>(logits, E, K, idx, w);
    else topk_wave<16>(logits, E, K, idx, w);
}

// Q8_1 quantization of `nblk` 32-blocks (ggml semantics, see quant.hip) by a
// 256-thread group, one half-wave per block.  src(b, i) is element i of block
// b; emit(b, i, q, d, sum) receives the block's results (every lane gets d
// and sum).
template <class Src, class Emit>
__device__ __forceinline__ void quantize_blocks(int nblk, Src src, Emit emit) {
    for (int b = threadIdx.x >> 5; b < nblk; b += GEMV_THREADS / 32) {
        const int i = threadIdx.x & 31;
        const float xi = src(b, i);
        const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        emit(b, i, q, d, sum);
    }
}

}  // namespace chimere
