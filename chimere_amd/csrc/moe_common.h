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
// multiply-add, then tree_sum256 (NT > 1: the NT trees side by side, red of
// NT * 256 floats).  Results valid in thread 0.
template <int NT>
__device__ __forceinline__ void f32_row_dot(const float* __restrict__ a, const float* __restrict__ x,
                                            int H, int ntok, float* red, float (&out)[NT]) {
    constexpr int U = 8;   // columns per thread loaded together before use
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
    for (int j0 = threadIdx.x; j0 < H; j0 += 256 * U) {
        // every load of the step is issued before any is used (tokens past
        // ntok re-read the last token; their sums are not returned)
        float av[U], xv[NT][U];
#pragma unroll
        for (int u = 0; u < U; u++) av[u] = j0 + 256 * u < H ? a[j0 + 256 * u] : 0.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int64_t tt = t < ntok ? t : ntok - 1;
#pragma unroll
            for (int u = 0; u < U; u++) xv[t][u] = j0 + 256 * u < H ? x[tt * H + j0 + 256 * u] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int u = 0; u < U; u++)
                if (j0 + 256 * u < H) acc[t] = __builtin_fmaf(av[u], xv[t][u], acc[t]);
    }
    if constexpr (NT == 1) {
        out[0] = tree_sum256(acc[0], red);
    } else {
        // the NT trees side by side: red holds NT * 256 floats
        const int tid = threadIdx.x;
#pragma unroll
        for (int t = 0; t < NT; t++) red[t * 256 + tid] = acc[t];
        __syncthreads();
        if (tid < 128)
#pragma unroll
            for (int t = 0; t < NT; t++) red[t * 256 + tid] = red[t * 256 + tid] + red[t * 256 + tid + 128];
        __syncthreads();
        if (tid < 64) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                float w = red[t * 256 + tid] + red[t * 256 + tid + 64];
                w = w + xlane<32>(w);
                out[t] = bfly32_sum(w);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- top-k

// Fast exact selection of the K largest of 4 keys per lane (E <= 256,
// K <= 16), wave-local through `sc` (128 u64 of LDS owned by this wave; a
// wave's LDS accesses complete in issue order, so no barrier is needed).
// Composite c = key << 32 | ~index orders entries as the k rounds of arg-max
// do (larger p first, lower index on equal p); all composites differ.
//  1. candidates: the entries with key >= a threshold, the largest of eight
//     fractions of the top probability for which at least K entries pass
//     (each count is four ballots and their population counts, scalar work
//     with no cross-lane chain); every entry above a candidate is a
//     candidate, so a candidate's round is the number of candidates above it;
//  2. the n candidates (K <= n <= 64) are compacted into sc[64..64+n) in
//     index order (slot-major offsets from the ballots' population counts
//     and each lane's count of set bits below it), and lane l < n counts the
//     candidates above candidate l;
//  3. the candidate of round r is written to sc[r]; lane k < K takes round
//     k and every lane sums rounds 0..K-1 in order (the renormalisation sum).
// Returns false (nothing written) when no threshold leaves between K and 64
// candidates (e.g. many exactly equal probabilities): the caller then runs
// the k rounds of arg-max.  Otherwise lane k < K gets round k's index and
// renormalised weight in my_idx / my_w.
__device__ __forceinline__ bool topk4_select(const uint32_t (&key)[4], uint32_t kmax, int K, uint64_t* sc,
                                             int& my_idx, float& my_w) {
    const int lane = threadIdx.x & 63;
    const float pmax = __builtin_bit_cast(float, kmax - 1u);
    constexpr float FR[8] = {0.7f, 0.5f, 0.35f, 0.25f, 0.17f, 0.12f, 0.08f, 0.05f};
    uint32_t thr = 0;
    int n = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const uint32_t kt = __builtin_bit_cast(uint32_t, pmax * FR[t]) + 1u;
        int c = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) c += __builtin_popcountll(__ballot(key[i] >= kt));
        if (c >= K) { thr = kt; n = c; break; }
    }
    if (n < K || n > 64) return false;
    int base = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint64_t m = __ballot(key[i] >= thr);
        if (key[i] >= thr) {
            const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            sc[64 + pos] = ((uint64_t)key[i] << 32) | (uint32_t)~(uint32_t)(lane + 64 * i);
        }
        base += __builtin_popcountll(m);
    }
    if (lane >= n) sc[64 + lane] = 0;   // below every composite
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const ulonglong2* c2p = (const ulonglong2*)(sc + 64);
    const uint64_t mine = sc[64 + lane];
    int r0 = 0, r1 = 0;
    for (int j0 = 0; j0 < n; j0 += 8) {   // chunks of 8 candidates (the zeros past n count nothing)
        ulonglong2 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = c2p[j0 / 2 + j];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            r0 += v[j].x > mine ? 1 : 0;
            r1 += v[j].y > mine ? 1 : 0;
        }
    }
    const int rank = r0 + r1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < n && rank < K) sc[rank] = mine;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float ws = 0.0f, w = 0.0f;
    int id = 0;
    for (int k0 = 0; k0 < K; k0 += 8) {
        uint64_t r[8];
#pragma unroll
        for (int k = 0; k < 8; k++) r[k] = sc[k0 + k];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k0 + k < K) {
                const float p = __builtin_bit_cast(float, (uint32_t)(r[k] >> 32) - 1u);
                ws += p;
                if (k0 + k == lane) { w = p; id = (int)~(uint32_t)r[k]; }
            }
        }
    }
    my_idx = id;
    my_w = ws > 0.0f ? w * (1.0f / ws) : w;
    __builtin_amdgcn_wave_barrier();
    return true;
}

// Softmax + top-k + renormalisation of one logits row by ONE wavefront, in
// registers (cs/kernels/chimere_kernels.cu:1150-1223): lane l holds logits
// l, l+64, ... (NV = ceil(E/64) values, zero-padded).  p = exp(l - max) / sum
// where the sum follows the reference's strided halving tree (strides
// 512..64 pair values inside a lane, strides 32..1 pair lanes; padding adds
// +0, which leaves the non-negative partial sums unchanged).
// Selection: the reference takes k rounds of arg-max by probability with ties
// to the lowest index; so does this, in registers: a round takes the wave
// maximum of the keys f32bits(p) + 1 (0 marks a taken or padding entry; p >= 0
// so the key order is the order of p; keys < 2^31) by a DPP scan, the lowest index
// holding it (ballots of key == max, slot by slot), and clears that entry.  Weights are
// renormalised by the sequential sum of the selected probabilities (round
// order).  Lane k < K writes entry k.  Requires E <= 1024, K <= min(E, 64).
// With `sc` (128 u64 of the wave's LDS), 128 < E <= 256 and K <= 16, the
// selection and renormalisation run as topk4_select above (same results).
template <int NV>
__device__ __forceinline__ void topk_wave(const float* __restrict__ logits, int E, int K,
                                          int* __restrict__ idx_out, float* __restrict__ w_out,
                                          uint64_t* sc = nullptr) {
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
    uint32_t key[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = lane + 64 * i;
        p[i] = s > 0.0f ? ev[i] / s : 1.0f / (float)E;
        key[i] = j < E ? __builtin_bit_cast(uint32_t, p[i]) + 1u : 0u;
    }
    int my_idx = 0;
    float my_w = 0.0f;
    bool fast = false;
    if constexpr (NV == 4) {
      // the top key: p_max = 1 / s (the maximum's exponential is exactly 1)
      const uint32_t kmax = __builtin_bit_cast(uint32_t, s > 0.0f ? 1.0f / s : 1.0f / (float)E) + 1u;
      fast = sc != nullptr && K <= 16 && topk4_select(key, kmax, K, sc, my_idx, my_w);
      if (!fast) {
        // Each lane's keys sorted once, descending, equal keys by index (the
        // order (key, -index) is total, so any sorting network gives it).
        // A round is then a maximum over the lanes' heads: the winner is the
        // lane whose head holds it (the lowest index among several such
        // lanes: a slow path for exact ties), which then pops its head.
        uint32_t kk[4] = {key[0], key[1], key[2], key[3]};
        int sl[4] = {0, 1, 2, 3};
        auto cx = [&](int a, int b) {
            const bool sw = kk[b] > kk[a] || (kk[b] == kk[a] && sl[b] < sl[a]);
            const uint32_t ka = kk[a], kb = kk[b];
            const int sa = sl[a], sb = sl[b];
            kk[a] = sw ? kb : ka;
            kk[b] = sw ? ka : kb;
            sl[a] = sw ? sb : sa;
            sl[b] = sw ? sa : sb;
        };
        cx(0, 1);
        cx(2, 3);
        cx(0, 2);
        cx(1, 3);
        cx(1, 2);
        for (int k = 0; k < K; k++) {
            const int m = wave_max_nonneg((int)kk[0]);
            const uint64_t bm = __ballot(kk[0] == (uint32_t)m);
            int wl;
            if (__builtin_popcountll(bm) == 1) {
                wl = __builtin_ctzll(bm);
            } else {
                const int cand = kk[0] == (uint32_t)m ? 0x7FFFFFFF - (lane + 64 * sl[0]) : 0;
                wl = (0x7FFFFFFF - wave_max_nonneg(cand)) & 63;
            }
            const int win = __builtin_amdgcn_readlane(lane + 64 * sl[0], wl);
            if (lane == wl) {
                kk[0] = kk[1]; kk[1] = kk[2]; kk[2] = kk[3]; kk[3] = 0u;
                sl[0] = sl[1]; sl[1] = sl[2]; sl[2] = sl[3];
            }
            if (lane == k) { my_idx = win; my_w = __builtin_bit_cast(float, (uint32_t)m - 1u); }
        }
      }
    } else
    for (int k = 0; k < K; k++) {
        int m = (int)key[0];
#pragma unroll
        for (int i = 1; i < NV; i++) m = max(m, (int)key[i]);
        m = wave_max_nonneg(m);
        // the lowest index holding m: indices of slot i (lane + 64 i) all
        // precede those of slot i + 1, so it is the lowest lane of the first
        // slot whose ballot of key == m is not empty
        int win = 0;
        bool found = false;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint64_t bm = __ballot(key[i] == (uint32_t)m);
            if (!found && bm != 0) {
                win = 64 * i + __builtin_ctzll(bm);
                found = true;
            }
        }
        win = __builtin_amdgcn_readfirstlane(win);
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (lane + 64 * i == win) key[i] = 0u;
        if (lane == k) { my_idx = win; my_w = __builtin_bit_cast(float, (uint32_t)m - 1u); }
    }
    if (!fast) {
        float ws = 0.0f;
        for (int k = 0; k < K; k++)
            ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), k));
        my_w = ws > 0.0f ? my_w * (1.0f / ws) : my_w;
    }
    if (lane < K) {
        idx_out[lane] = my_idx;
        w_out[lane] = my_w;
    }
}

// E outside (128, 256]: out of line, so that the common case's code stays
// compact in the instruction cache
static __device__ __noinline__ void topk_wave_other(const float* logits, int E, int K, int* idx, float* w) {
    if (E <= 64) topk_wave<1>(logits, E, K, idx, w);
    else if (E <= 128) topk_wave<2>(logits, E, K, idx, w);
    else if (E <= 512) topk_wave<8>(logits, E, K, idx, w);
    else topk_wave<16>(logits, E, K, idx, w);
}

// sc: 128 u64 of LDS owned by the calling wave (the fast selection for
// 128 < E <= 256), or nullptr
__device__ __forceinline__ void topk_wave_any(const float* logits, int E, int K, int* idx, float* w,
                                              uint64_t* sc = nullptr) {
    if (E > 128 && E <= 256) topk_wave<4>(logits, E, K, idx, w, sc);
    else topk_wave_other(logits, E, K, idx, w);
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
