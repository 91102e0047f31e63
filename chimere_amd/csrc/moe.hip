// moe.hip -- routed MoE FFN layer for 1..8 decode tokens, plus the
// standalone router / top-k / elementwise kernels of the reference's MoE
// glue (cs/src/kernels/{elementwise,topk_softmax,fused_ops}.rs,
// cs/src/scratch_pool.rs).
//
// Layer = 3 launches on the caller's stream:
//   K1 k_moe_route    one work-group per router row (+1 for the shared-expert
//                     gate vector): f32 logits for every token; the last
//                     work-group to finish (ticket counter) runs softmax/top-k
//                     per token, quantizes x to Q8_1 and builds the list of
//                     distinct selected experts with their (token, k) pairs.
//   K2 k_moe_gate_up  (8-row chunk of F) x (distinct expert | shared): 8 gate
//                     rows + 8 up rows per 16-row tile, each weight byte read
//                     once for all tokens routed to the expert; h =
//                     silu(gate)*up; the last of the four work-groups covering
//                     a 32-row block quantizes it to Q8_1.
//   K3 k_moe_down     16 hidden rows per work-group over all selected experts
//                     (tiles of several experts staged together), then the
//                     router-weighted sum in k order plus the shared expert.
// Every row dot uses the (L=16, G=1) order of tile_gemv.h.  Ticket counters
// return to zero before each kernel exits.
#include "api_internal.h"
#include "common.h"
#include "tile_gemv.h"

namespace chimere {

__constant__ uint32_t c_iq3s_grid_moe[512] = CHIMERE_IQ3S_GRID_INIT;

constexpr int MAX_TOK = 8;
constexpr int MAX_K = 16;
constexpr int MAX_E = 1024;
constexpr int DOWN_LDS_BUDGET = 40 * 1024;

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
        w = w + __shfl_xor(w, 32);
        w = w + __shfl_xor(w, 16);
        w = w + __shfl_xor(w, 8);
        w = w + __shfl_xor(w, 4);
        w = w + __shfl_xor(w, 2);
        w = w + __shfl_xor(w, 1);
        v = w;
    }
    __syncthreads();
    return v;
}

__device__ __forceinline__ float block_max256(float v, float* red) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m));
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    v = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

// f32 row dot of `a` (H) against NT tokens of x (token stride H), in the
// reference's order: thread t accumulates columns t, t+256, ... with fused
// multiply-add, then tree_sum256.  Results valid in thread 0.
template <int NT>
__device__ __forceinline__ void f32_row_dot(const float* __restrict__ a, const float* __restrict__ x,
                                            int H, int ntok, float* red, float (&out)[NT]) {
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
    for (int j = threadIdx.x; j < H; j += 256) {
        const float av = a[j];
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (t < ntok) acc[t] = __builtin_fmaf(av, x[(int64_t)t * H + j], acc[t]);
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
        if (t < ntok) out[t] = tree_sum256(acc[t], red);
}

// ---------------------------------------------------------------- top-k

// Softmax + top-k + renormalisation of one logits row by a 256-thread group
// (cs/kernels/chimere_kernels.cu:1150-1223): p = exp(l - max) / sum with the
// sum taken by the strided halving tree; k rounds of arg-max by probability
// (ties -> lowest index); weights renormalised by the sequential sum of the
// selected probabilities.  `logits` may be in global memory; lp/lev are LDS
// scratch of E floats.
__device__ void topk_group(const float* logits, int E, int K, int* idx, float* w,
                           float* lp, float* lev, float* red, int* redi) {
    const int tid = threadIdx.x;
    float mx = -__builtin_huge_valf();
    for (int i = tid; i < E; i += 256) mx = __builtin_fmaxf(mx, logits[i]);
    mx = block_max256(mx, red);
    for (int i = tid; i < E; i += 256) {
        const float e = det_exp(logits[i] - mx);
        lev[i] = e;
        lp[i] = e;
    }
    __syncthreads();
    for (int st = 512; st >= 1; st >>= 1) {
        for (int t = tid; t < st; t += 256)
            if (t + st < E) lp[t] = lp[t] + lp[t + st];
        __syncthreads();
    }
    const float sum = lp[0];
    __syncthreads();
    for (int i = tid; i < E; i += 256) lp[i] = sum > 0.0f ? lev[i] / sum : 1.0f / (float)E;
    __syncthreads();
    for (int k = 0; k < K; k++) {
        float bv = -2.0f;
        int bi = 0x7fffffff;
        for (int i = tid; i < E; i += 256)
            if (lp[i] > bv) { bv = lp[i]; bi = i; }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m);
            const int oi = __shfl_xor(bi, m);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if ((tid & 63) == 0) { red[tid >> 6] = bv; redi[tid >> 6] = bi; }
        __syncthreads();
        if (tid == 0) {
            for (int q = 1; q < 4; q++)
                if (red[q] > bv || (red[q] == bv && redi[q] < bi)) { bv = red[q]; bi = redi[q]; }
            idx[k] = bi;
            w[k] = bv;
            lp[bi] = -1.0f;
        }
        __syncthreads();
    }
    if (tid == 0) {
        float ws = 0.0f;
        for (int k = 0; k < K; k++) ws += w[k];
        if (ws > 0.0f) {
            const float inv = 1.0f / ws;
            for (int k = 0; k < K; k++) w[k] = w[k] * inv;
        }
    }
    __syncthreads();
}

// Q8_1 quantization of `nblk` 32-blocks (ggml semantics, see quant.hip) by a
// 256-thread group, one half-wave per block.  src(b, i) is element i of block
// b; dst(b) is the 36-byte output block.
template <class Src, class Dst>
__device__ __forceinline__ void quantize_blocks(int nblk, Src src, Dst dst) {
    for (int b = threadIdx.x >> 5; b < nblk; b += 8) {
        const int i = threadIdx.x & 31;
        const float xi = src(b, i);
        float amax = __builtin_fabsf(xi), sum = xi;
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) {
            amax = __builtin_fmaxf(amax, __shfl_xor(amax, m, 32));
            sum = sum + __shfl_xor(sum, m, 32);
        }
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* blk = dst(b);
        blk[4 + i] = (uint8_t)(int8_t)q;
        if (i == 0) *(uint32_t*)blk = f2h(d) | (f2h(sum) << 16);
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
    int* route_cnt;     // [1]
    int* gu_cnt;        // [(M*K+1) * F/32]
    float* logits;      // [M*E]
    float* glogit;      // [M]
    int* ids;           // [M*K]
    float* wts;         // [M*K]
    int* n_unique;      // [1]
    int* uexp;          // [M*K]
    int* u_ntok;        // [M*K]
    int* u_pair;        // [M*K][MAX_TOK]  pair = t*K + k
    int* u_tok;         // [M*K][MAX_TOK]
    uint8_t* xq;        // [M][xq_stride]
    float* h;           // [M*K + M][F]
    uint8_t* hq;        // [M*K + M][hq_stride]
    int64_t xq_stride, hq_stride;
};

__global__ __launch_bounds__(256) void k_moe_route(MoeArgs a) {
    __shared__ float red[256];
    __shared__ int redi[4];
    __shared__ int ticket;
    __shared__ float lp[MAX_E], lev[MAX_E];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    float v[MAX_TOK];
    const float* A = row < a.E ? a.router + (int64_t)row * a.H : a.sh_gate_w;
    f32_row_dot<MAX_TOK>(A, a.x, a.H, a.M, red, v);
    if (tid == 0) {
        for (int t = 0; t < a.M; t++) {
            if (row < a.E) a.logits[t * a.E + row] = a.bias ? v[t] + a.bias[row] : v[t];
            else a.glogit[t] = v[t];
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) ticket = atomicAdd(a.route_cnt, 1);
    __syncthreads();
    if (ticket != (int)gridDim.x - 1) return;
    __threadfence();
    // ---- last work-group: routing for every token, Q8_1(x), expert plan
    for (int t = 0; t < a.M; t++) {
        topk_group(a.logits + t * a.E, a.E, a.K, a.ids + t * a.K, a.wts + t * a.K, lp, lev, red, redi);
    }
    {
        const int nbpr = a.H / QK;
        quantize_blocks(
            a.M * nbpr,
            [&](int b, int i) { return a.x[(int64_t)(b / nbpr) * a.H + (b % nbpr) * QK + i]; },
            [&](int b) { return a.xq + (int64_t)(b / nbpr) * a.xq_stride + (int64_t)(b % nbpr) * Q8_1_BYTES; });
    }
    if (tid == 0) {
        int* map = (int*)lp;   // reuse: expert -> distinct index
        for (int e = 0; e < a.E; e++) map[e] = -1;
        int nu = 0;
        for (int t = 0; t < a.M; t++)
            for (int k = 0; k < a.K; k++) {
                const int e = a.ids[t * a.K + k];
                int u = map[e];
                if (u < 0) { u = nu++; map[e] = u; a.uexp[u] = e; a.u_ntok[u] = 0; }
                const int n = a.u_ntok[u]++;
                a.u_pair[u * MAX_TOK + n] = t * a.K + k;
                a.u_tok[u * MAX_TOK + n] = t;
            }
        *a.n_unique = nu;
        if (a.ids_out)
            for (int i = 0; i < a.M * a.K; i++) { a.ids_out[i] = a.ids[i]; a.w_out[i] = a.wts[i]; }
        *a.route_cnt = 0;
    }
}

// K2: grid (F/8, M*K + 1).  blockIdx.y < n_unique: routed expert; == M*K: shared.
template <int TE, int TS>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_gate_up(MoeArgs a) {
    constexpr int CBE = ChunkGeom<TE>::BYTES, CBS = ChunkGeom<TS>::BYTES;
    constexpr int CB = CBE > CBS ? CBE : CBS;
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE_ROWS * CB + 16];
    __shared__ XLds xs[MAX_TOK][CHUNK_BLOCKS];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ float res[TILE_ROWS][MAX_TOK];
    __shared__ int toks[MAX_TOK], pairs[MAX_TOK];
    __shared__ int ticket;

    const int u = blockIdx.y;
    const bool shared = u == a.M * a.K;
    if (shared ? !a.has_shared : u >= *a.n_unique) return;
    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * 8;
    int ntok;
    if (shared) {
        ntok = a.M;
        if (tid < a.M) { toks[tid] = tid; pairs[tid] = a.M * a.K + tid; }
    } else {
        ntok = a.u_ntok[u];
        if (tid < ntok) { toks[tid] = a.u_tok[u * MAX_TOK + tid]; pairs[tid] = a.u_pair[u * MAX_TOK + tid]; }
    }
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_moe[i];

    float acc[MAX_TOK];
    if (shared) {
        const int64_t rb = row_bytes(TS, a.H);
        tile_gemv<TS, MAX_TOK>(tile, CB, xs, grid, a.sh_gate + r0 * rb, 8, a.sh_up + r0 * rb, 8, rb,
                               a.H, a.xq, a.xq_stride, toks, ntok, acc);
    } else {
        const int64_t rb = row_bytes(TE, a.H);
        const int64_t e = a.uexp[u];
        tile_gemv<TE, MAX_TOK>(tile, CB, xs, grid, a.gate + e * a.sg + r0 * rb, 8,
                               a.up + e * a.su + r0 * rb, 8, rb, a.H, a.xq, a.xq_stride, toks, ntok, acc);
    }
    const int g = tid >> 4, j = tid & 15;
#pragma unroll
    for (int t = 0; t < MAX_TOK; t++) {
        const float v = slot_reduce16(acc[t]);
        if (j == 0 && t < ntok) res[g][t] = v;
    }
    __syncthreads();
    if (tid < 8 * ntok) {
        const int i = tid & 7, t = tid >> 3;
        const float hv = det_silu(res[i][t]) * res[8 + i][t];
        a.h[(int64_t)pairs[t] * a.F + r0 + i] = hv;
    }
    __threadfence();
    __syncthreads();
    int* cnt = a.gu_cnt + (int64_t)u * (a.F / QK) + r0 / QK;
    if (tid == 0) ticket = atomicAdd(cnt, 1);
    __syncthreads();
    if (ticket != QK / 8 - 1) return;
    __threadfence();
    // last of the 4 work-groups of this 32-row block: quantize h for each token
    const int blk = r0 / QK;
    if ((tid >> 5) < ntok) {
        const int t = tid >> 5, i = tid & 31;
        const float* hp = a.h + (int64_t)pairs[t] * a.F + blk * QK;
        const float xi = __hip_atomic_load(hp + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float amax = __builtin_fabsf(xi), sum = xi;
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) {
            amax = __builtin_fmaxf(amax, __shfl_xor(amax, m, 32));
            sum = sum + __shfl_xor(sum, m, 32);
        }
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* o = a.hq + (int64_t)pairs[t] * a.hq_stride + blk * Q8_1_BYTES;
        o[4 + i] = (uint8_t)(int8_t)q;
        if (i == 0) *(uint32_t*)o = f2h(d) | (f2h(sum) << 16);
    }
    if (tid == 0) *cnt = 0;
}

// Down-projection rows of one expert tile (in LDS) for the given pairs; writes
// dn[pair][row] for the 16 rows.  F <= 64 blocks (one chunk).
template <int T>
__device__ __forceinline__ void down_tile(const uint8_t* tile, int lstride, const uint32_t* grid,
                                          const uint8_t* hq, int64_t hq_stride, int F,
                                          const int* pairs, int np, int nr, float (*dn)[TILE_ROWS]) {
    const int tid = threadIdx.x, g = tid >> 4, j = tid & 15;
    const int nb = F / QK;
    const uint8_t* row = tile + g * lstride;
    for (int p = 0; p < np; p++) {
        float acc = 0.0f;
        if (g < nr) {
            for (int b = j; b < nb; b += SLOTS) {
                XBlk xb;
                load_xblk(hq + (int64_t)pairs[p] * hq_stride + (int64_t)b * Q8_1_BYTES, xb);
                float dw;
                const int s = block_dot<T>(row, b, xb, grid, &dw);
                acc = __builtin_fmaf(dw * xb.d, (float)s, acc);
            }
            const float v = slot_reduce16(acc);
            if (j == 0) dn[pairs[p]][g] = v;
        }
    }
}

// K3: grid (ceil(H/16)).
template <int TE, int TS>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_down(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t tiles[DOWN_LDS_BUDGET + 16];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ float dn[MAX_TOK * MAX_K + MAX_TOK][TILE_ROWS];
    __shared__ int pl[MAX_TOK * MAX_K + 1][MAX_TOK];
    __shared__ int np[MAX_TOK * MAX_K + 1];
    __shared__ int wexp[MAX_TOK * MAX_K + 1];

    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * TILE_ROWS;
    const int nr = min(TILE_ROWS, a.H - r0);
    const int nu = *a.n_unique;
    const int nw = nu + (a.has_shared ? 1 : 0);
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_moe[i];
    for (int w = tid; w < nw; w += GEMV_THREADS) {
        if (w < nu) {
            wexp[w] = a.uexp[w];
            np[w] = a.u_ntok[w];
            for (int i = 0; i < np[w]; i++) pl[w][i] = a.u_pair[w * MAX_TOK + i];
        } else {
            wexp[w] = -1;
            np[w] = a.M;
            for (int i = 0; i < a.M; i++) pl[w][i] = a.M * a.K + i;
        }
    }
    const int64_t rbE = row_bytes(TE, a.F), rbS = row_bytes(TS, a.F);
    const int lsE = (int)((rbE + 15) & ~15), lsS = (int)((rbS + 15) & ~15);
    int w0 = 0;
    while (w0 < nw) {
        // choose a batch of work experts whose tiles fit in LDS
        int w1 = w0, used = 0;
        while (w1 < nw) {
            const int need = TILE_ROWS * ((w1 < nu) ? lsE : lsS);
            if (used + need > DOWN_LDS_BUDGET && w1 > w0) break;
            used += need;
            w1++;
        }
        __syncthreads();
        int off = 0;
        for (int w = w0; w < w1; w++) {
            if (w < nu) {
                stage_rows(tiles + off, lsE, a.down + (int64_t)wexp[w] * a.sd + (int64_t)r0 * rbE, rbE, nr,
                           (int)rbE, tid, GEMV_THREADS);
                off += TILE_ROWS * lsE;
            } else {
                stage_rows(tiles + off, lsS, a.sh_down + (int64_t)r0 * rbS, rbS, nr, (int)rbS, tid,
                           GEMV_THREADS);
                off += TILE_ROWS * lsS;
            }
        }
        __syncthreads();
        off = 0;
        for (int w = w0; w < w1; w++) {
            if (w < nu) {
                down_tile<TE>(tiles + off, lsE, grid, a.hq, a.hq_stride, a.F, pl[w], np[w], nr, dn);
                off += TILE_ROWS * lsE;
            } else {
                down_tile<TS>(tiles + off, lsS, grid, a.hq, a.hq_stride, a.F, pl[w], np[w], nr, dn);
                off += TILE_ROWS * lsS;
            }
        }
        w0 = w1;
    }
    __syncthreads();
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
}

// ------------------------------------------------------- workspace plan

struct WsPlan {
    size_t route_cnt, gu_cnt, logits, glogit, ids, wts, n_unique, uexp, u_ntok, u_pair, u_tok, xq, h, hq, total;
    int64_t xq_stride, hq_stride;
};

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

static WsPlan plan_ws(int H, int F, int E, int K, int M) {
    WsPlan p{};
    size_t o = 0;
    const int P = M * K + M;
    p.xq_stride = pad_to(H, ROW_PAD) / QK * Q8_1_BYTES;
    p.hq_stride = pad_to(F, ROW_PAD) / QK * Q8_1_BYTES;
    p.route_cnt = o; o += al256(4);
    p.gu_cnt = o; o += al256((size_t)(M * K + 1) * (F / QK) * 4);
    p.logits = o; o += al256((size_t)M * E * 4);
    p.glogit = o; o += al256((size_t)M * 4);
    p.ids = o; o += al256((size_t)M * K * 4);
    p.wts = o; o += al256((size_t)M * K * 4);
    p.n_unique = o; o += al256(4);
    p.uexp = o; o += al256((size_t)M * K * 4);
    p.u_ntok = o; o += al256((size_t)M * K * 4);
    p.u_pair = o; o += al256((size_t)M * K * MAX_TOK * 4);
    p.u_tok = o; o += al256((size_t)M * K * MAX_TOK * 4);
    p.xq = o; o += al256((size_t)M * p.xq_stride);
    p.h = o; o += al256((size_t)P * F * 4);
    p.hq = o; o += al256((size_t)P * p.hq_stride);
    p.total = o;
    return p;
}

// stage < 0: all three kernels; 0, 1, 2: only K1, K2 or K3
template <int TE, int TS>
static void launch_layer(const MoeArgs& a, int stage, hipStream_t s) {
    if (stage < 0 || stage == 0)
        hipLaunchKernelGGL(k_moe_route, dim3(a.E + (a.sh_gate_w ? 1 : 0)), dim3(256), 0, s, a);
    if (stage < 0 || stage == 1)
        hipLaunchKernelGGL((k_moe_gate_up<TE, TS>), dim3(a.F / 8, a.M * a.K + 1), dim3(GEMV_THREADS), 0, s, a);
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

__global__ __launch_bounds__(256) void k_topk(const float* logits, int* idx, float* w, int E, int K) {
    __shared__ float red[256];
    __shared__ int redi[4];
    __shared__ float lp[MAX_E], lev[MAX_E];
    __shared__ int sidx[MAX_K * 64];
    __shared__ float sw[MAX_K * 64];
    const int t = blockIdx.x;
    topk_group(logits + (int64_t)t * E, E, K, sidx, sw, lp, lev, red, redi);
    for (int k = threadIdx.x; k < K; k += 256) { idx[t * K + k] = sidx[k]; w[t * K + k] = sw[k]; }
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
    CHIMERE_REQUIRE(E >= 1 && E <= MAX_E && K >= 1 && K <= MAX_K && K <= E, CHIMERE_ERR_ARG,
                    "moe_ffn_decode: n_experts=%d top_k=%d out of range", E, K);
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
    a.route_cnt = (int*)(w + p.route_cnt); a.gu_cnt = (int*)(w + p.gu_cnt);
    a.logits = (float*)(w + p.logits); a.glogit = (float*)(w + p.glogit);
    a.ids = (int*)(w + p.ids); a.wts = (float*)(w + p.wts);
    a.n_unique = (int*)(w + p.n_unique); a.uexp = (int*)(w + p.uexp); a.u_ntok = (int*)(w + p.u_ntok);
    a.u_pair = (int*)(w + p.u_pair); a.u_tok = (int*)(w + p.u_tok);
    a.xq = w + p.xq; a.h = (float*)(w + p.h); a.hq = w + p.hq;
    a.xq_stride = p.xq_stride; a.hq_stride = p.hq_stride;
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
    CHIMERE_REQUIRE(E >= 1 && E <= MAX_E && K >= 1 && K <= E && K <= MAX_K * 64 && ntok >= 1, CHIMERE_ERR_ARG,
                    "topk_softmax: n_experts=%d top_k=%d ntok=%d out of range", E, K, ntok);
    hipLaunchKernelGGL(k_topk, dim3(ntok), dim3(256), 0, s, logits, idx, w, E, K);
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
