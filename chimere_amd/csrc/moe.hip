// moe.hip -- routed MoE FFN layer for 1..8 decode tokens, plus the
// standalone router / top-k / elementwise kernels of the reference's MoE
// glue (cs/src/kernels/{elementwise,topk_softmax,fused_ops}.rs,
// cs/src/scratch_pool.rs).
//
// Layer = 3 launches on the caller's stream; no work-group ever waits on
// another (kernel boundaries are the only synchronisation, so no device-scope
// fences or counters are needed):
//   K1 k_moe_route    one work-group per router row (+1 for the shared-expert
//                     gate vector) computing f32 logits for every token, plus
//                     one work-group per token quantizing x to Q8_1.
//   K2 k_moe_gate_up  (32-row block of F) x (distinct expert | shared).  Each
//                     routed work-group recomputes softmax/top-k (one wave per
//                     token, registers only) and the distinct-expert plan from
//                     the 1 KB of logits, then streams 32 gate + 32 up rows of
//                     its expert once for all tokens routed to it and writes
//                     the block of h = silu(gate)*up Q8_1-quantized.
//   K3 k_moe_down     16 hidden rows per work-group over all selected experts
//                     (tiles of several experts staged together with their
//                     Q8_1 intermediates), then the router-weighted sum in k
//                     order plus the shared expert.
// Every row dot uses the (L=16, G=1) order of tile_gemv.h.
#include "api_internal.h"
#include "common.h"
#include "tile_gemv.h"

// Phase timestamps for latency analysis (debug builds with
// -DCHIMERE_PHASE_TIMING only): thread 0 of a work-group records the 100 MHz
// real-time counter at numbered points into workspace.
#ifdef CHIMERE_PHASE_TIMING
#define PHASE(kern, i)                                                                      \
    do {                                                                                     \
        if (threadIdx.x == 0)                                                                \
            a.phase[((kern) * 4096 + blockIdx.x + blockIdx.y * gridDim.x) * 8 + (i)] =        \
                __builtin_amdgcn_s_memrealtime();                                           \
    } while (0)
#else
#define PHASE(kern, i) do {} while (0)
#endif

namespace chimere {

__constant__ uint32_t c_iq3s_grid_moe[512] = CHIMERE_IQ3S_GRID_INIT;

constexpr int MAX_TOK = 8;
constexpr int MAX_K = 16;
constexpr int MAX_E = 1024;        // standalone top-k
constexpr int MAX_E_FUSED = 256;   // fused MoE layer (one logit per thread of a 256-thread group)

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
    uint64_t T = 0;
    for (int b = 40; b >= 0; b--) {
        const uint64_t cand = T | (1ull << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NV; i++) cnt += __popcll(__ballot(key[i] >= cand));
        if (cnt >= K) T = cand;
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

// Softmax + top-k of one logits row (E <= 256) by a 256-thread group, with
// low dependent depth.  Thread i owns logit i (padding i >= E).  max: wave
// DPP butterflies + LDS; sum: the reference's strided halving tree (strides
// 128 and 64 through LDS, 32..1 by xor exchanges, which equal the tree at
// lane 0); p = ev / sum.  Selection: a bitonic sort, descending, of the
// 41-bit keys (f32 bits of p << 11 | 1024 - index) -- the same set and order
// as k rounds of arg-max with ties to the lowest index; strides >= 64 go
// through LDS, smaller ones are in-wave DPP / permlane exchanges.  The first
// K threads of the group then hold the result; weights are renormalised by
// the sequential sum of the selected probabilities.  `scr` is LDS scratch of
// 256 uint64 + 8 floats for this group; every thread of the work-group must
// call this the same number of times (it contains __syncthreads()).
__device__ __forceinline__ uint64_t xlane64(uint64_t v, int m) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    switch (m) {
    case 1: lo = xlane<1>((int)lo); hi = xlane<1>((int)hi); break;
    case 2: lo = xlane<2>((int)lo); hi = xlane<2>((int)hi); break;
    case 4: lo = xlane<4>((int)lo); hi = xlane<4>((int)hi); break;
    case 8: lo = xlane<8>((int)lo); hi = xlane<8>((int)hi); break;
    case 16: lo = xlane<16>((int)lo); hi = xlane<16>((int)hi); break;
    default: lo = xlane<32>((int)lo); hi = xlane<32>((int)hi); break;
    }
    return ((uint64_t)hi << 32) | lo;
}

__device__ void topk_block256(const float* __restrict__ logits, int E, int K, bool active, int* idx_out,
                              float* w_out, uint64_t* scr) {
    const int i = threadIdx.x & 255;
    const int wv = i >> 6;
    float* fs = (float*)(scr + 256);
    const float l = (active && i < E) ? logits[i] : -__builtin_huge_valf();
    float m = bfly32_max(__builtin_fmaxf(l, xlane<32>(l)));
    if ((i & 63) == 0) fs[wv] = m;
    __syncthreads();
    m = __builtin_fmaxf(__builtin_fmaxf(fs[0], fs[1]), __builtin_fmaxf(fs[2], fs[3]));
    const float ev = (active && i < E) ? det_exp(l - m) : 0.0f;
    float* ps = (float*)scr;
    ps[i] = ev;
    __syncthreads();
    if (i < 128) ps[i] = ps[i] + ps[i + 128];
    __syncthreads();
    float sum = 0.0f;
    if (i < 64) {
        float v = ps[i] + ps[i + 64];
        v = v + xlane<32>(v);
        sum = bfly32_sum(v);
        if (i == 0) fs[4] = sum;
    }
    __syncthreads();
    sum = fs[4];
    const float p = sum > 0.0f ? ev / sum : 1.0f / (float)E;
    uint64_t key = (active && i < E) ? (((uint64_t)__builtin_bit_cast(uint32_t, p)) << 11) | (uint64_t)(1024 - i) : 0;
    __syncthreads();   // ps (aliases scr) is free again
    for (int k = 2; k <= 256; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            uint64_t other;
            if (j >= 64) {
                scr[i] = key;
                __syncthreads();
                other = scr[i ^ j];
                __syncthreads();
            } else {
                other = xlane64(key, j);
            }
            const bool lower = (i & j) == 0;
            const bool desc = (i & k) == 0 || k == 256;
            const uint64_t mx = key > other ? key : other, mn = key > other ? other : key;
            key = (lower == desc) ? mx : mn;
        }
    }
    // threads 0..K-1 (wave 0 of the group) hold the K largest keys in order
    const uint32_t pb = (uint32_t)(key >> 11);
    const float pv = __builtin_bit_cast(float, pb);
    float ws = 0.0f;
    if (wv == 0) {
        for (int k = 0; k < K; k++) ws += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), k));
    }
    if (active && i < K) {
        idx_out[i] = 1024 - (int)(key & 0x7FF);
        w_out[i] = ws > 0.0f ? pv * (1.0f / ws) : pv;
    }
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

// ------------------------------------------------------------ MoE layer

struct MoeArgs {
    int H, F, E, K, M;
    int has_shared;
    const float* x;
    float* out;
    const float* router;
    const float* bias;
    const uint8_t *gate, *up, *down;
    int64_t sg, su, sd;
    const uint8_t *sh_gate, *sh_up, *sh_down;
    const float* sh_gate_w;
    int* ids_out;
    float* w_out;
    // workspace
    float* logits;      // [M*E]
    float* glogit;      // [M]
    float* wts;         // [M*K]
    int* plan;          // n_unique, uexp[128], u_ntok[128], u_pair[128][MAX_TOK]
    uint8_t* xq;        // [M][xq_stride]   Q8_1(x)
    uint8_t* hq;        // [M*K + M][hq_stride]   Q8_1(h) per (token, k) pair and shared
    int64_t xq_stride, hq_stride;
    uint64_t* phase;    // debug timestamps (CHIMERE_PHASE_TIMING builds)
};

constexpr int PLAN_UEXP = 1, PLAN_UNTOK = 1 + MAX_TOK * MAX_K, PLAN_UPAIR = 1 + 2 * MAX_TOK * MAX_K;
constexpr int PLAN_INTS = PLAN_UPAIR + MAX_TOK * MAX_K * MAX_TOK;

// Expert plan: distinct selected experts and, per expert, its (token, k) pairs.
struct Plan {
    int nu;
    int uexp[MAX_TOK * MAX_K];
    int untok[MAX_TOK * MAX_K];
    int upair[MAX_TOK * MAX_K][MAX_TOK];
    int utok[MAX_TOK * MAX_K][MAX_TOK];
};

// K1: grid E (router rows) + has_gate (shared-expert gate row) + M (x quantizers).
__global__ __launch_bounds__(256) void k_moe_route(MoeArgs a) {
    __shared__ float red[256];
    PHASE(0, 0);
    const int row = blockIdx.x;
    const int ng = a.sh_gate_w ? 1 : 0;
    if (row >= a.E + ng) {
        const int t = row - a.E - ng;
        const int nb = a.H / QK;
        const float* xt = a.x + (int64_t)t * a.H;
        uint8_t* dst = a.xq + t * a.xq_stride;
        quantize_blocks(
            nb, [&](int b, int i) { return xt[b * QK + i]; },
            [&](int b, int i, int q, float d, float sum) {
                uint8_t* blk = dst + b * Q8_1_BYTES;
                blk[4 + i] = (uint8_t)(int8_t)q;
                if (i == 0) *(uint32_t*)blk = f2h(d) | (f2h(sum) << 16);
            });
        return;
    }
    float v[MAX_TOK];
    const float* A = row < a.E ? a.router + (int64_t)row * a.H : a.sh_gate_w;
    f32_row_dot<MAX_TOK>(A, a.x, a.H, a.M, red, v);
    if (threadIdx.x == 0) {
        for (int t = 0; t < a.M; t++) {
            if (row < a.E) a.logits[t * a.E + row] = a.bias ? v[t] + a.bias[row] : v[t];
            else a.glogit[t] = v[t];
        }
    }
    PHASE(0, 1);
}

constexpr int GU_RG = 64;                  // K2 row groups: 1024 threads
constexpr int GU_THREADS = GU_RG * SLOTS;

// K2: grid (F/32, M*K + 1), 1024 threads.  Every routed work-group recomputes
// the routing (top-k per token, one wave each) and the distinct-expert plan
// from the logits, so no work-group waits on another; blockIdx.y < n_unique
// selects a distinct expert, blockIdx.y == M*K the shared expert.  Work-group
// (0,0) publishes routing and plan for K3.  A tile holds 32 gate + 32 up rows
// (group g < 32 computes gate row g, group 32 + g up row g), so the
// work-group owns whole 32-row blocks of h = silu(gate) * up and writes them
// Q8_1-quantized.
template <int TE, int TS>
__global__ __launch_bounds__(GU_THREADS) void k_moe_gate_up(MoeArgs a) {
    constexpr int CBE = ChunkGeom<TE>::BYTES, CBS = ChunkGeom<TS>::BYTES;
    constexpr int CB = CBE > CBS ? CBE : CBS;
    // the tile buffer first holds the expert map and the plan (routing phase)
    constexpr int ROUTE_BYTES = MAX_E_FUSED * 4 + (int)sizeof(Plan) + 4 * (256 + 32) * 8;
    constexpr int TILE_BYTES = GU_RG * CB + 16 > ROUTE_BYTES ? GU_RG * CB + 16 : ROUTE_BYTES;
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE_BYTES];
    __shared__ XLds xs[MAX_TOK][MAX_CHUNK_BLOCKS];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ float hg[MAX_TOK][QK], hu[MAX_TOK][QK];
    __shared__ int toks[MAX_TOK], pairs[MAX_TOK];
    __shared__ int s_ids[MAX_TOK * MAX_K];
    __shared__ float s_w[MAX_TOK * MAX_K];
    Plan& pl = *(Plan*)(tile + MAX_E_FUSED * 4);
    uint64_t* tscr = (uint64_t*)(tile + MAX_E_FUSED * 4 + sizeof(Plan));

    const int u = blockIdx.y;
    const bool shared = u == a.M * a.K;
    const int tid = threadIdx.x;
    PHASE(1, 0);
    if (shared && !a.has_shared) return;
    int ntok;
    if (shared) {
        ntok = a.M;
        if (tid < a.M) { toks[tid] = tid; pairs[tid] = a.M * a.K + tid; }
    } else {
        const int grp = tid >> 8;   // four 256-thread groups, one token each per pass
        for (int t0 = 0; t0 < a.M; t0 += GU_THREADS / 256) {
            const int t = t0 + grp;
            const bool act = t < a.M;
            topk_block256(a.logits + (act ? t : 0) * a.E, a.E, a.K, act, s_ids + (act ? t : 0) * a.K,
                          s_w + (act ? t : 0) * a.K, tscr + grp * (256 + 32));
        }
        __syncthreads();
        int* map = (int*)tile;
        for (int e = tid; e < a.E; e += GU_THREADS) map[e] = -1;
        __syncthreads();
        PHASE(1, 1);
        if (tid == 0) {
            int nu = 0;
            for (int t = 0; t < a.M; t++)
                for (int k = 0; k < a.K; k++) {
                    const int e = s_ids[t * a.K + k];
                    int uu = map[e];
                    if (uu < 0) { uu = nu++; map[e] = uu; pl.uexp[uu] = e; pl.untok[uu] = 0; }
                    const int n = pl.untok[uu]++;
                    pl.upair[uu][n] = t * a.K + k;
                    pl.utok[uu][n] = t;
                }
            pl.nu = nu;
        }
        __syncthreads();
        if (blockIdx.x == 0 && u == 0) {
            const int nu = pl.nu;
            for (int i = tid; i < a.M * a.K; i += GU_THREADS) {
                a.wts[i] = s_w[i];
                if (a.ids_out) { a.ids_out[i] = s_ids[i]; a.w_out[i] = s_w[i]; }
            }
            int* P = a.plan;
            if (tid == 0) P[0] = nu;
            for (int i = tid; i < nu; i += GU_THREADS) {
                P[PLAN_UEXP + i] = pl.uexp[i];
                P[PLAN_UNTOK + i] = pl.untok[i];
                for (int n = 0; n < pl.untok[i]; n++) P[PLAN_UPAIR + i * MAX_TOK + n] = pl.upair[i][n];
            }
        }
        if (u >= pl.nu) return;
        ntok = pl.untok[u];
        if (tid < ntok) { toks[tid] = pl.utok[u][tid]; pairs[tid] = pl.upair[u][tid]; }
    }
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += GU_THREADS) grid[i] = c_iq3s_grid_moe[i];
    PHASE(1, 2);
    const int r0 = blockIdx.x * QK;
    float acc[1][MAX_TOK];
    if (shared) {
        const int64_t rb = row_bytes(TS, a.H);
        tile_gemv<TS, MAX_TOK, GU_RG, 1>(tile, xs, grid, a.sh_gate + r0 * rb, QK, a.sh_up + r0 * rb, QK, rb,
                                         a.H, a.xq, a.xq_stride, toks, ntok, acc);
    } else {
        const int64_t rb = row_bytes(TE, a.H);
        const int64_t e = pl.uexp[u];
        tile_gemv<TE, MAX_TOK, GU_RG, 1>(tile, xs, grid, a.gate + e * a.sg + r0 * rb, QK,
                                         a.up + e * a.su + r0 * rb, QK, rb, a.H, a.xq, a.xq_stride, toks,
                                         ntok, acc);
    }
    PHASE(1, 3);
    const int g = tid >> 4, j = tid & 15;
#pragma unroll
    for (int t = 0; t < MAX_TOK; t++) {
        if (t < ntok) {
            const float v = slot_reduce16(acc[0][t]);
            if (j == 0) {
                if (g < QK) hg[t][g] = v;
                else hu[t][g - QK] = v;
            }
        }
    }
    __syncthreads();
    // one half-wave per token quantizes the 32-row block of h (ggml Q8_1)
    if ((tid >> 5) < ntok) {
        const int t = tid >> 5, i = tid & 31;
        const float xi = det_silu(hg[t][i]) * hu[t][i];
        const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* o = a.hq + (int64_t)pairs[t] * a.hq_stride + blockIdx.x * Q8_1_BYTES;
        o[4 + i] = (uint8_t)(int8_t)q;
        if (i == 0) *(uint32_t*)o = f2h(d) | (f2h(sum) << 16);
    }
    PHASE(1, 4);
}

// Down-projection rows of one expert tile (in LDS) for its pairs, with the
// pairs' Q8_1 intermediates decoded in LDS (xl[p][block]); writes
// dn[pair][row] for the tile's rows.
template <int T>
__device__ __forceinline__ void down_tile(const uint8_t* tile, int lstride, const uint32_t* grid,
                                          const XLds* xl, int nbF, const int* pairs, int np, int nr,
                                          float (*dn)[TILE_ROWS]) {
    const int tid = threadIdx.x, g = tid >> 4, j = tid & 15;
    const uint8_t* row = tile + g * lstride;
    for (int p = 0; p < np; p++) {
        float acc = 0.0f;
        if (g < nr) {
            for (int b = j; b < nbF; b += SLOTS) {
                XBlk xb;
                xlds_to_blk(xl[p * nbF + b], xb);
                float dw;
                const int s = block_dot<T>(row, b, xb, grid, &dw);
                acc = __builtin_fmaf(dw * xb.d, (float)s, acc);
            }
            const float v = slot_reduce16(acc);
            if (j == 0) dn[pairs[p]][g] = v;
        }
    }
}

constexpr int DOWN_LDS = 96 * 1024;

// K3: grid (ceil(H/16)), 256 threads.  Stages the down tiles of a batch of
// experts together with their pairs' Q8_1 intermediates (decoded into LDS),
// computes, then combines in k order plus the shared expert.
template <int TE, int TS>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_down(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t buf[DOWN_LDS + 16];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ float dn[MAX_TOK * MAX_K + MAX_TOK][TILE_ROWS];
    __shared__ int pl[MAX_TOK * MAX_K + 1][MAX_TOK];
    __shared__ int np[MAX_TOK * MAX_K + 1];
    __shared__ int wexp[MAX_TOK * MAX_K + 1];
    __shared__ int boff[MAX_TOK * MAX_K + 1], xoff[MAX_TOK * MAX_K + 1];

    const int tid = threadIdx.x;
    PHASE(2, 0);
    const int r0 = blockIdx.x * TILE_ROWS;
    const int nr = min(TILE_ROWS, a.H - r0);
    const int* P = a.plan;
    const int nu = P[0];
    const int nw = nu + (a.has_shared ? 1 : 0);
    const int nbF = a.F / QK;
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_moe[i];
    for (int w = tid; w < nw; w += GEMV_THREADS) {
        if (w < nu) {
            wexp[w] = P[PLAN_UEXP + w];
            np[w] = P[PLAN_UNTOK + w];
            for (int i = 0; i < np[w]; i++) pl[w][i] = P[PLAN_UPAIR + w * MAX_TOK + i];
        } else {
            wexp[w] = -1;
            np[w] = a.M;
            for (int i = 0; i < a.M; i++) pl[w][i] = a.M * a.K + i;
        }
    }
    __syncthreads();
    PHASE(2, 1);
    const int64_t rbE = row_bytes(TE, a.F), rbS = row_bytes(TS, a.F);
    const int lsE = (int)rbE, lsS = (int)rbS;   // tiles packed with the row stride
    int w0 = 0;
    while (w0 < nw) {
        // a batch of work experts whose tiles and decoded intermediates fit in LDS
        int w1 = w0, used = 0;
        while (w1 < nw) {
            const int need = ((TILE_ROWS * ((w1 < nu) ? lsE : lsS) + 15) & ~15) + np[w1] * nbF * (int)sizeof(XLds);
            if (used + need > DOWN_LDS && w1 > w0) break;
            used += need;
            w1++;
        }
        {
            int o = 0;
            for (int w = w0; w < w1; w++) { if (tid == 0) boff[w] = o; o += (TILE_ROWS * ((w < nu) ? lsE : lsS) + 15) & ~15; }
            for (int w = w0; w < w1; w++) { if (tid == 0) xoff[w] = o; o += np[w] * nbF * (int)sizeof(XLds); }
        }
        __syncthreads();
        for (int w = w0; w < w1; w++) {
            if (w < nu)
                stage_rows(buf + boff[w], a.down + (int64_t)wexp[w] * a.sd + (int64_t)r0 * rbE, rbE, nr, (int)rbE,
                           tid, GEMV_THREADS);
            else
                stage_rows(buf + boff[w], a.sh_down + (int64_t)r0 * rbS, rbS, nr, (int)rbS, tid, GEMV_THREADS);
        }
        // decode every pair's Q8_1 intermediate of the batch in one parallel pass
        // (xoff of consecutive work experts is contiguous, so block i of the batch
        // lands at xoff[w0] + i)
        {
            int tot = 0;
            for (int w = w0; w < w1; w++) tot += np[w] * nbF;
            XLds* xl = (XLds*)(buf + xoff[w0]);
            for (int i = tid; i < tot; i += GEMV_THREADS) {
                int w = w0, r = i;
                while (r >= np[w] * nbF) { r -= np[w] * nbF; w++; }
                XBlk xb;
                load_xblk(a.hq + (int64_t)pl[w][r / nbF] * a.hq_stride + (int64_t)(r % nbF) * Q8_1_BYTES, xb);
#pragma unroll
                for (int k = 0; k < 8; k++) xl[i].q[k] = xb.q[k];
                xl[i].d = xb.d;
                xl[i].sumq = xb.sumq;
            }
        }
        PHASE(2, 2);
        lds_copy_wait();
        __syncthreads();
        PHASE(2, 3);
        for (int w = w0; w < w1; w++) {
            const XLds* xl = (const XLds*)(buf + xoff[w]);
            if (w < nu) down_tile<TE>(buf + boff[w], lsE, grid, xl, nbF, pl[w], np[w], nr, dn);
            else down_tile<TS>(buf + boff[w], lsS, grid, xl, nbF, pl[w], np[w], nr, dn);
        }
        __syncthreads();
        PHASE(2, 4);
        w0 = w1;
    }
    // combine: acc = sum_k fmaf(w_k, dn_k, acc); out = fmaf(shared, sigmoid(g), acc)
    if (tid < a.M * TILE_ROWS) {
        const int t = tid / TILE_ROWS, r = tid % TILE_ROWS;
        if (r < nr) {
            float acc = 0.0f;
            for (int k = 0; k < a.K; k++) acc = __builtin_fmaf(a.wts[t * a.K + k], dn[t * a.K + k][r], acc);
            float o = acc;
            if (a.has_shared) {
                const float sh = dn[a.M * a.K + t][r];
                if (a.sh_gate_w) {
                    const float sc = 1.0f / (1.0f + det_exp(-a.glogit[t]));
                    o = __builtin_fmaf(sh, sc, acc);
                } else {
                    o = sh + acc;
                }
            }
            a.out[(int64_t)t * a.H + r0 + r] = o;
        }
    }
    PHASE(2, 5);
}

// ------------------------------------------------------- workspace plan

struct WsPlan {
    size_t logits, glogit, wts, plan, xq, hq, phase, total;
    int64_t xq_stride, hq_stride;
};

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

static WsPlan plan_ws(int H, int F, int E, int K, int M) {
    WsPlan p{};
    size_t o = 0;
    const int P = M * K + M;
    p.xq_stride = pad_to(H, ROW_PAD) / QK * Q8_1_BYTES;
    p.hq_stride = pad_to(F, ROW_PAD) / QK * Q8_1_BYTES;
    p.logits = o; o += al256((size_t)M * E * 4);
    p.glogit = o; o += al256((size_t)M * 4);
    p.wts = o; o += al256((size_t)M * K * 4);
    p.plan = o; o += al256((size_t)PLAN_INTS * 4);
    p.xq = o; o += al256((size_t)M * p.xq_stride);
    p.hq = o; o += al256((size_t)P * p.hq_stride);
#ifdef CHIMERE_PHASE_TIMING
    p.phase = o; o += al256((size_t)3 * 4096 * 8 * 8);
#endif
    p.total = o;
    return p;
}

// stage < 0: all three kernels; 0, 1, 2: only K1, K2 or K3
template <int TE, int TS>
static void launch_layer(const MoeArgs& a, int stage, hipStream_t s) {
    if (stage < 0 || stage == 0)
        hipLaunchKernelGGL(k_moe_route, dim3(a.E + (a.sh_gate_w ? 1 : 0) + a.M), dim3(256), 0, s, a);
    if (stage < 0 || stage == 1)
        hipLaunchKernelGGL((k_moe_gate_up<TE, TS>), dim3(a.F / QK, a.M * a.K + 1), dim3(GU_THREADS), 0, s, a);
    if (stage < 0 || stage == 2)
        hipLaunchKernelGGL((k_moe_down<TE, TS>), dim3((a.H + TILE_ROWS - 1) / TILE_ROWS), dim3(GEMV_THREADS), 0,
                           s, a);
}

template <int TE>
static bool dispatch_ts(int ts, const MoeArgs& a, int stage, hipStream_t s) {
    switch (ts) {
    case T_Q8_0: launch_layer<TE, T_Q8_0>(a, stage, s); return true;
    case T_Q4_0: launch_layer<TE, T_Q4_0>(a, stage, s); return true;
    case T_IQ3_S: launch_layer<TE, T_IQ3_S>(a, stage, s); return true;
    }
    return false;
}

static bool dispatch_layer(int te, int ts, const MoeArgs& a, int stage, hipStream_t s) {
    if (ts < 0) ts = te;
    switch (te) {
    case T_Q8_0: return dispatch_ts<T_Q8_0>(ts, a, stage, s);
    case T_Q4_0: return dispatch_ts<T_Q4_0>(ts, a, stage, s);
    case T_IQ3_S: return dispatch_ts<T_IQ3_S>(ts, a, stage, s);
    }
    return false;
}

static bool valid_type(int t) { return t == T_Q8_0 || t == T_Q4_0 || t == T_IQ3_S; }

// ---------------------------------------------- standalone glue kernels

__global__ __launch_bounds__(256) void k_f32_gemv(const float* A, const float* x, float* y, int cols) {
    __shared__ float red[256];
    float v[1];
    f32_row_dot<1>(A + (int64_t)blockIdx.x * cols, x, cols, 1, red, v);
    if (threadIdx.x == 0) y[blockIdx.x] = v[0];
}

__global__ __launch_bounds__(64) void k_topk(const float* logits, int* idx, float* w, int E, int K) {
    const int t = blockIdx.x;
    topk_wave_any(logits + (int64_t)t * E, E, K, idx + t * K, w + t * K);
}

__global__ void k_silu_mul(float* g, const float* u, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) g[i] = det_silu(g[i]) * u[i];
}

__global__ void k_weighted_combine(const float* eo, const float* w, float* acc, int H, int K) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    float s = 0.0f;
    for (int k = 0; k < K; k++) s = __builtin_fmaf(w[k], eo[(int64_t)k * H + i], s);
    acc[i] = s;
}

__global__ void k_sigmoid_gate_add(float* out, const float* gate, const float* comb, int n) {
    const float sc = 1.0f / (1.0f + det_exp(-gate[0]));
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __builtin_fmaf(out[i], sc, comb[i]);
}

__global__ void k_fill_zero(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace chimere

using namespace chimere;

extern "C" {

size_t chimere_moe_workspace_size(const chimere_moe_layer* L, int max_ntok) {
    if (!L || max_ntok < 1 || max_ntok > MAX_TOK) return 0;
    return plan_ws(L->hidden, L->ffn, L->n_experts, L->top_k, max_ntok).total;
}

void chimere_moe_workspace_init(void* ws, size_t bytes, hipStream_t s) {
    CHIMERE_REQUIRE(ws && bytes % 4 == 0, CHIMERE_ERR_ARG, "moe_workspace_init: bad workspace");
    hipLaunchKernelGGL(k_fill_zero, dim3(256), dim3(256), 0, s, (uint32_t*)ws, bytes / 4);
    check_launch("moe_workspace_init");
}

static void moe_decode(const chimere_moe_layer* L, const float* x, float* out, int ntok, int* ids_out,
                       float* w_out, void* workspace, size_t ws_bytes, int stage, hipStream_t stream) {
    CHIMERE_REQUIRE(L && x && out && workspace, CHIMERE_ERR_ARG, "moe_ffn_decode: null pointer");
    const int H = L->hidden, F = L->ffn, E = L->n_experts, K = L->top_k;
    CHIMERE_REQUIRE(ntok >= 1 && ntok <= MAX_TOK, CHIMERE_ERR_ARG, "moe_ffn_decode: ntok=%d not in 1..8", ntok);
    CHIMERE_REQUIRE(H > 0 && H % 256 == 0 && F > 0 && F % 256 == 0 && F <= 2048, CHIMERE_ERR_ARG,
                    "moe_ffn_decode: hidden=%d / ffn=%d must be multiples of 256 (ffn <= 2048)", H, F);
    CHIMERE_REQUIRE(E >= 1 && E <= MAX_E_FUSED && K >= 1 && K <= MAX_K && K <= E, CHIMERE_ERR_ARG,
                    "moe_ffn_decode: n_experts=%d (<= 256) top_k=%d (<= 16) out of range", E, K);
    CHIMERE_REQUIRE(valid_type(L->expert_type), CHIMERE_ERR_ARG, "moe_ffn_decode: expert_type %d", L->expert_type);
    const bool has_sh = L->shared_type >= 0;
    CHIMERE_REQUIRE(!has_sh || (valid_type(L->shared_type) && L->sh_gate && L->sh_up && L->sh_down),
                    CHIMERE_ERR_ARG, "moe_ffn_decode: shared expert incomplete");
    CHIMERE_REQUIRE(L->router_w && L->gate_exps && L->up_exps && L->down_exps, CHIMERE_ERR_ARG,
                    "moe_ffn_decode: null weight pointer");
    CHIMERE_REQUIRE(!ids_out == !w_out, CHIMERE_ERR_ARG, "moe_ffn_decode: ids_out and w_out go together");
    const int64_t rbH = row_bytes(L->expert_type, H), rbF = row_bytes(L->expert_type, F);
    CHIMERE_REQUIRE(L->gate_stride >= rbH * F && L->up_stride >= rbH * F && L->down_stride >= rbF * H,
                    CHIMERE_ERR_ARG, "moe_ffn_decode: expert strides too small");
    CHIMERE_REQUIRE((((uintptr_t)L->gate_exps | (uintptr_t)L->up_exps | (uintptr_t)L->down_exps |
                      (uintptr_t)L->gate_stride | (uintptr_t)L->up_stride | (uintptr_t)L->down_stride) & 1) == 0,
                    CHIMERE_ERR_ARG, "moe_ffn_decode: weights must be 2-byte aligned");
    const WsPlan p = plan_ws(H, F, E, K, ntok);
    CHIMERE_REQUIRE(ws_bytes >= p.total && ((uintptr_t)workspace & 255) == 0, CHIMERE_ERR_WORKSPACE,
                    "moe_ffn_decode: workspace %zu bytes < %zu (or not 256-byte aligned)", ws_bytes, p.total);
    uint8_t* w = (uint8_t*)workspace;
    MoeArgs a{};
    a.H = H; a.F = F; a.E = E; a.K = K; a.M = ntok;
    a.has_shared = has_sh;
    a.x = x; a.out = out; a.router = L->router_w; a.bias = L->logit_bias;
    a.gate = (const uint8_t*)L->gate_exps; a.up = (const uint8_t*)L->up_exps; a.down = (const uint8_t*)L->down_exps;
    a.sg = L->gate_stride; a.su = L->up_stride; a.sd = L->down_stride;
    a.sh_gate = (const uint8_t*)L->sh_gate; a.sh_up = (const uint8_t*)L->sh_up; a.sh_down = (const uint8_t*)L->sh_down;
    a.sh_gate_w = has_sh ? L->sh_gate_w : nullptr;
    a.ids_out = ids_out; a.w_out = w_out;
    a.logits = (float*)(w + p.logits); a.glogit = (float*)(w + p.glogit);
    a.wts = (float*)(w + p.wts); a.plan = (int*)(w + p.plan);
    a.xq = w + p.xq; a.hq = w + p.hq;
    a.xq_stride = p.xq_stride; a.hq_stride = p.hq_stride;
    a.phase = (uint64_t*)(w + p.phase);
    dispatch_layer(L->expert_type, L->shared_type, a, stage, stream);
    check_launch("moe_ffn_decode");
}

void chimere_moe_ffn_decode(const chimere_moe_layer* L, const float* x, float* out, int ntok,
                            int* ids_out, float* w_out, void* workspace, size_t ws_bytes,
                            hipStream_t stream) {
    moe_decode(L, x, out, ntok, ids_out, w_out, workspace, ws_bytes, -1, stream);
}

void chimere_moe_ffn_decode_stage(const chimere_moe_layer* L, const float* x, float* out, int ntok,
                                  void* workspace, size_t ws_bytes, int stage, hipStream_t stream) {
    CHIMERE_REQUIRE(stage >= -1 && stage <= 2, CHIMERE_ERR_ARG, "moe_ffn_decode_stage: stage %d", stage);
    moe_decode(L, x, out, ntok, nullptr, nullptr, workspace, ws_bytes, stage, stream);
}

void chimere_f32_gemv(const float* A, const float* x, float* y, int rows, int cols, hipStream_t s) {
    CHIMERE_REQUIRE(A && x && y && rows > 0 && cols > 0, CHIMERE_ERR_ARG, "f32_gemv: bad arguments");
    hipLaunchKernelGGL(k_f32_gemv, dim3(rows), dim3(256), 0, s, A, x, y, cols);
    check_launch("f32_gemv");
}

void chimere_topk_softmax(const float* logits, int* idx, float* w, int E, int K, int ntok, hipStream_t s) {
    CHIMERE_REQUIRE(logits && idx && w, CHIMERE_ERR_ARG, "topk_softmax: null pointer");
    CHIMERE_REQUIRE(E >= 1 && E <= MAX_E && K >= 1 && K <= E && K <= MAX_K && ntok >= 1, CHIMERE_ERR_ARG,
                    "topk_softmax: n_experts=%d top_k=%d ntok=%d out of range", E, K, ntok);
    hipLaunchKernelGGL(k_topk, dim3(ntok), dim3(64), 0, s, logits, idx, w, E, K);
    check_launch("topk_softmax");
}

void chimere_silu_mul_inplace(float* g, const float* u, int n, hipStream_t s) {
    CHIMERE_REQUIRE(g && u && n > 0, CHIMERE_ERR_ARG, "silu_mul: bad arguments");
    hipLaunchKernelGGL(k_silu_mul, dim3((n + 255) / 256), dim3(256), 0, s, g, u, n);
    check_launch("silu_mul");
}

void chimere_weighted_combine(const float* eo, const float* w, float* acc, int H, int K, hipStream_t s) {
    CHIMERE_REQUIRE(eo && w && acc && H > 0 && K > 0, CHIMERE_ERR_ARG, "weighted_combine: bad arguments");
    hipLaunchKernelGGL(k_weighted_combine, dim3((H + 255) / 256), dim3(256), 0, s, eo, w, acc, H, K);
    check_launch("weighted_combine");
}

void chimere_sigmoid_gate_add(float* out, const float* gate, const float* comb, int n, hipStream_t s) {
    CHIMERE_REQUIRE(out && gate && comb && n > 0, CHIMERE_ERR_ARG, "sigmoid_gate_add: bad arguments");
    hipLaunchKernelGGL(k_sigmoid_gate_add, dim3((n + 255) / 256), dim3(256), 0, s, out, gate, comb, n);
    check_launch("sigmoid_gate_add");
}

}  // extern "C"
