// prefill.hip -- routed MoE FFN for a chunk of tokens (prefill): tokens are
// routed, grouped by expert, and each expert's gate/up and down projections
// run as int8 MFMA grouped GEMMs (v_mfma_i32_32x32x32_i8: one 32-element
// quantization block per instruction, so every block's int32 dot is exact),
// with the per-block fp32 rescale acc = fmaf(f32(d_w) * f32(d_x), (float)sumi,
// acc) applied in ascending block order (the L=1 order).  No counterpart in
// the reference, which runs its decode MoE once per prompt token
// (cs/src/qwen35_model/compute_graph.rs:1787-1800); the per-token arithmetic
// is that of cs/src/qwen35_model/moe_ffn.rs:1081-1768.
//
// Launches: P1 router logits (reference order) + Q8_1(x); P2 softmax/top-k
// per token; P3 expert plan (counting sort of (token, k) pairs by expert,
// 32-pair tiles); P4 gate/up MFMA + silu*up + Q8_1(h); P5 down MFMA; P6
// router-weighted sum in k order plus the shared expert.
#include "api_internal.h"
#include "common.h"
#include "moe_common.h"

namespace chimere {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int PF_CHUNK = 8;      // 32-element blocks per K chunk staged in LDS
constexpr int PF_TILE = 32;      // (token, k) pairs per MFMA tile (the M dimension)
constexpr int PF_THREADS = 256;  // 4 waves

struct PfArgs {
    int H, F, E, K, T, has_shared;
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
    float* logits;   // [T][E]
    float* glogit;   // [T]
    int* ids;        // [T*K]
    float* wts;      // [T*K]
    uint8_t* xq;     // [T][xq_stride]
    int* off;        // [E+2] start of each expert's pairs in spairs
    int* spairs;     // [T*K + T] pairs grouped by expert (shared expert last)
    int* tiles;      // [max_tiles][3] (expert, start, count)
    int* ntiles;     // [1]
    uint8_t* hq;     // [T*K + T][hq_stride] Q8_1(h) per pair
    float* dn;       // [T*K + T][H] down-projection output per pair
    int64_t xq_stride, hq_stride;
    int max_tiles;
};

// P1: grid (E + has_gate, ceil(T/8)): router logits for 8 tokens per work-group.
__global__ __launch_bounds__(256) void k_pf_router(PfArgs a) {
    __shared__ float red[256];
    const int row = blockIdx.x, t0 = blockIdx.y * MAX_TOK;
    const int nt = min(MAX_TOK, a.T - t0);
    float v[MAX_TOK];
    const float* A = row < a.E ? a.router + (int64_t)row * a.H : a.sh_gate_w;
    f32_row_dot<MAX_TOK>(A, a.x + (int64_t)t0 * a.H, a.H, nt, red, v);
    if (threadIdx.x == 0)
        for (int t = 0; t < nt; t++) {
            if (row < a.E) a.logits[(int64_t)(t0 + t) * a.E + row] = a.bias ? v[t] + a.bias[row] : v[t];
            else a.glogit[t0 + t] = v[t];
        }
}

// P2: one wave per token
__global__ __launch_bounds__(64) void k_pf_topk(PfArgs a) {
    const int t = blockIdx.x;
    topk_wave_any(a.logits + (int64_t)t * a.E, a.E, a.K, a.ids + t * a.K, a.wts + t * a.K);
}

// P3: one work-group.  Counting sort of the T*K pairs by expert (the order of
// pairs inside an expert does not affect any result: every pair's output row
// is computed on its own), the shared expert as expert E with all T tokens,
// and the list of 32-pair tiles.
__global__ __launch_bounds__(1024) void k_pf_plan(PfArgs a) {
    __shared__ int cnt[MAX_E + 1], fill[MAX_E + 1], off[MAX_E + 2];
    const int tid = threadIdx.x, TK = a.T * a.K, NE = a.E + 1;
    for (int e = tid; e < NE; e += 1024) { cnt[e] = 0; fill[e] = 0; }
    __syncthreads();
    for (int p = tid; p < TK; p += 1024) atomicAdd(&cnt[a.ids[p]], 1);
    if (tid == 0) cnt[a.E] = a.has_shared ? a.T : 0;
    __syncthreads();
    if (tid == 0) {
        int o = 0, nt = 0;
        for (int e = 0; e < NE; e++) {
            off[e] = o;
            for (int s = 0; s < cnt[e]; s += PF_TILE) {
                a.tiles[nt * 3] = e;
                a.tiles[nt * 3 + 1] = o + s;
                a.tiles[nt * 3 + 2] = min(PF_TILE, cnt[e] - s);
                nt++;
            }
            o += cnt[e];
        }
        off[NE] = o;
        *a.ntiles = nt;
    }
    __syncthreads();
    for (int e = tid; e <= NE; e += 1024) a.off[e] = off[e];
    for (int p = tid; p < TK; p += 1024) {
        const int e = a.ids[p];
        a.spairs[off[e] + atomicAdd(&fill[e], 1)] = p;
        if (a.ids_out) { a.ids_out[p] = e; a.w_out[p] = a.wts[p]; }
    }
    if (a.has_shared)
        for (int t = tid; t < a.T; t += 1024) a.spairs[off[a.E] + t] = TK + t;
}

// ---- MFMA fragments.  v_mfma_i32_32x32x32_i8 layout: lane l supplies row
// l%32 of A and column l%32 of B, elements 16*(l/32) .. +16 of the K=32
// block; result D[i] at lane l is (row 8*(i/4) + 4*(l/32) + i%4, col l%32).

// 16 activation quants of a decoded Q8_1 block in LDS (q bytes at +4)
__device__ __forceinline__ v4i a_frag(const uint8_t* blk, int half) {
    const uint32_t* w = (const uint32_t*)(blk + 4 + 16 * half);
    v4i r;
    r.x = (int)w[0]; r.y = (int)w[1]; r.z = (int)w[2]; r.w = (int)w[3];
    return r;
}

// 16 weight values of a block row in LDS, as int8; Q4_0 gives the unsigned
// nibbles (0..15), corrected by -8 * sum(q_x) after the MFMA
template <int T>
__device__ __forceinline__ v4i b_frag(const uint8_t* row, int b, int half, float* dw) {
    v4i r;
    if constexpr (T == T_Q4_0) {
        const int off = b * 18;
        *dw = h2f(lds_u16(row, off));
        const int sh = 4 * half;
        r.x = (int)((lds_u32(row, off + 2) >> sh) & 0x0F0F0F0Fu);
        r.y = (int)((lds_u32(row, off + 6) >> sh) & 0x0F0F0F0Fu);
        r.z = (int)((lds_u32(row, off + 10) >> sh) & 0x0F0F0F0Fu);
        r.w = (int)((lds_u32(row, off + 14) >> sh) & 0x0F0F0F0Fu);
    } else {
        const int off = b * 34;
        *dw = h2f(lds_u16(row, off));
        const int q = off + 2 + 16 * half;
        r.x = (int)lds_u32(row, q);
        r.y = (int)lds_u32(row, q + 4);
        r.z = (int)lds_u32(row, q + 8);
        r.w = (int)lds_u32(row, q + 12);
    }
    return r;
}

// Stages, for one K chunk: `nrows` weight rows (global stride rb, chunk bytes
// cbytes at goff) into wlds, and the chunk of the tile's Q8_1 rows (src row
// stride xstride, 36*PF_CHUNK bytes at xoff) into xlds.
__device__ __forceinline__ void pf_stage(uint8_t* wlds, const uint8_t* w, int64_t rb, int nrows, int cbytes,
                                         uint8_t* xlds, const uint8_t* xsrc, const int* xrows, int64_t xstride,
                                         int64_t xoff) {
    stage_rows(wlds, w, rb, nrows, cbytes, threadIdx.x, PF_THREADS);
    // Q8_1 rows of the tile: 288 bytes each (18 pieces of 16 B), row index per pair
    constexpr int PER = 36 * PF_CHUNK / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int c0 = wave * 64; c0 < PF_TILE * PER; c0 += 4 * 64) {
        const int c = c0 + lane;
        if (c < PF_TILE * PER) {
            const int r = c / PER, col = c - r * PER;
            __builtin_amdgcn_global_load_lds((const glb_void_t*)(xsrc + xrows[r] * xstride + xoff + col * 16),
                                             (lds_void_t*)(xlds + c0 * 16), 16, 0, 0);
        }
    }
}

// 8 * sum of the 32 quants and f32(d) of every Q8_1 block in xlds
__device__ __forceinline__ void pf_xmeta(const uint8_t* xlds, int* xs8, float* xd) {
    const int i = threadIdx.x;   // PF_TILE * PF_CHUNK = 256 blocks, one per thread
    const uint8_t* blk = xlds + i * 36;
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) s = dot4(*(const int*)(blk + 4 + 4 * k), 0x01010101, s);
    xs8[i] = 8 * s;
    xd[i] = h2f(*(const uint16_t*)blk);
}

// One K chunk of a wave's 32x32 output tile: rows = pairs (A from xlds),
// columns = its 32 weight rows (B from wrows, row stride cbytes).
template <int T>
__device__ __forceinline__ void pf_mma_chunk(const uint8_t* xlds, const int* xs8, const float* xd,
                                             const uint8_t* wrows, int cbytes, int nb, float (&acc)[16]) {
    const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31;
    const uint8_t* wrow = wrows + col * cbytes;
    for (int b = 0; b < nb; b++) {
        float dw;
        const v4i bf = b_frag<T>(wrow, b, half, &dw);
        const v4i af = a_frag(xlds + ((lane & 31) * PF_CHUNK + b) * 36, half);
        v16i c = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, c, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int m = 8 * (i >> 2) + 4 * half + (i & 3);
            int s = c[i];
            if constexpr (T == T_Q4_0) s -= xs8[m * PF_CHUNK + b];
            acc[i] = __builtin_fmaf(dw * xd[m * PF_CHUNK + b], (float)s, acc[i]);
        }
    }
}

// P4: grid (F/64, max_tiles).  Waves 0,1: gate/up rows f0..f0+31; waves 2,3:
// gate/up rows f0+32..f0+63; then h = silu(gate)*up and Q8_1 of its two
// 32-row blocks per pair.
template <int TE, int TS>
__global__ __launch_bounds__(PF_THREADS) void k_pf_gate_up(PfArgs a) {
    constexpr int WB = (QTraits<TE>::BYTES > QTraits<TS>::BYTES ? QTraits<TE>::BYTES : QTraits<TS>::BYTES);
    __shared__ __attribute__((aligned(16))) uint8_t wlds[128 * PF_CHUNK * WB + 16];
    __shared__ __attribute__((aligned(16))) uint8_t xlds[PF_TILE * PF_CHUNK * 36 + 16];
    __shared__ int xs8[PF_TILE * PF_CHUNK];
    __shared__ float xd[PF_TILE * PF_CHUNK];
    __shared__ int prs[PF_TILE], xrows[PF_TILE];
    __shared__ float gu[2][PF_TILE][64];
    const int ti = blockIdx.y;
    if (ti >= *a.ntiles) return;
    const int e = a.tiles[ti * 3], start = a.tiles[ti * 3 + 1], n = a.tiles[ti * 3 + 2];
    const int tid = threadIdx.x, TK = a.T * a.K;
    if (tid < PF_TILE) {
        const int p = a.spairs[start + min(tid, n - 1)];   // padding rows repeat the last pair
        prs[tid] = p;
        xrows[tid] = p < TK ? p / a.K : p - TK;
    }
    const bool sh = e == a.E;
    const int f0 = blockIdx.x * 64;
    const int wave = tid >> 6, mat = wave & 1, rh = wave >> 1;
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    const int nbk = a.H / QK;
    auto run = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        const int64_t rb = row_bytes(T, a.H);
        const uint8_t* g = sh ? a.sh_gate : a.gate + (int64_t)e * a.sg;
        const uint8_t* u = sh ? a.sh_up : a.up + (int64_t)e * a.su;
        const int cbytes = PF_CHUNK * QTraits<T>::BYTES;
        for (int b0 = 0; b0 < nbk; b0 += PF_CHUNK) {
            __syncthreads();
            const int64_t goff = (int64_t)b0 * QTraits<T>::BYTES;
            stage_rows(wlds, g + f0 * rb + goff, rb, 64, cbytes, tid, PF_THREADS);
            pf_stage(wlds + 64 * cbytes, u + f0 * rb + goff, rb, 64, cbytes, xlds, a.xq, xrows, a.xq_stride,
                     (int64_t)b0 * 36);
            lds_copy_wait();
            __syncthreads();
            pf_xmeta(xlds, xs8, xd);
            __syncthreads();
            pf_mma_chunk<T>(xlds, xs8, xd, wlds + (mat * 64 + rh * 32) * cbytes, cbytes, PF_CHUNK, acc);
        }
    };
    if (sh) {
        if constexpr (TS == T_Q4_0) run(std::integral_constant<int, T_Q4_0>{});
        else run(std::integral_constant<int, T_Q8_0>{});
    } else {
        if constexpr (TE == T_Q4_0) run(std::integral_constant<int, T_Q4_0>{});
        else run(std::integral_constant<int, T_Q8_0>{});
    }
    {
        const int lane = tid & 63, half = lane >> 5, col = lane & 31;
#pragma unroll
        for (int i = 0; i < 16; i++) gu[mat][8 * (i >> 2) + 4 * half + (i & 3)][rh * 32 + col] = acc[i];
    }
    __syncthreads();
    // Q8_1(h) of the two 32-row blocks for each pair: one half-wave per (pair, block)
    for (int q = tid >> 5; q < 2 * n; q += PF_THREADS / 32) {
        const int m = q >> 1, blk = q & 1, i = tid & 31;
        const float xi = det_silu(gu[0][m][blk * 32 + i]) * gu[1][m][blk * 32 + i];
        const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
        const float d = amax / 127.0f;
        const int qv = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* o = a.hq + (int64_t)prs[m] * a.hq_stride + (f0 / QK + blk) * Q8_1_BYTES;
        o[4 + i] = (uint8_t)(int8_t)qv;
        if (i == 0) *(uint32_t*)o = f2h(d) | (f2h(sum) << 16);
    }
}

// P5: grid (H/128, max_tiles).  Wave w: down rows r0 + 32w .. +31 for the
// tile's 32 pairs; K = F.
template <int TE, int TS>
__global__ __launch_bounds__(PF_THREADS) void k_pf_down(PfArgs a) {
    constexpr int WB = (QTraits<TE>::BYTES > QTraits<TS>::BYTES ? QTraits<TE>::BYTES : QTraits<TS>::BYTES);
    __shared__ __attribute__((aligned(16))) uint8_t wlds[128 * PF_CHUNK * WB + 16];
    __shared__ __attribute__((aligned(16))) uint8_t xlds[PF_TILE * PF_CHUNK * 36 + 16];
    __shared__ int xs8[PF_TILE * PF_CHUNK];
    __shared__ float xd[PF_TILE * PF_CHUNK];
    __shared__ int prs[PF_TILE];
    const int ti = blockIdx.y;
    if (ti >= *a.ntiles) return;
    const int e = a.tiles[ti * 3], start = a.tiles[ti * 3 + 1], n = a.tiles[ti * 3 + 2];
    const int tid = threadIdx.x;
    if (tid < PF_TILE) prs[tid] = a.spairs[start + min(tid, n - 1)];
    const bool sh = e == a.E;
    const int r0 = blockIdx.x * 128, wave = tid >> 6;
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    const int nbk = a.F / QK;
    auto run = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        const int64_t rb = row_bytes(T, a.F);
        const uint8_t* d = sh ? a.sh_down : a.down + (int64_t)e * a.sd;
        for (int b0 = 0; b0 < nbk; b0 += PF_CHUNK) {
            const int cb = min(PF_CHUNK, nbk - b0);
            const int cbytes = cb * QTraits<T>::BYTES;
            __syncthreads();
            pf_stage(wlds, d + r0 * rb + (int64_t)b0 * QTraits<T>::BYTES, rb, 128, cbytes, xlds, a.hq, prs,
                     a.hq_stride, (int64_t)b0 * 36);
            lds_copy_wait();
            __syncthreads();
            pf_xmeta(xlds, xs8, xd);
            __syncthreads();
            pf_mma_chunk<T>(xlds, xs8, xd, wlds + wave * 32 * cbytes, cbytes, cb, acc);
        }
    };
    if (sh) {
        if constexpr (TS == T_Q4_0) run(std::integral_constant<int, T_Q4_0>{});
        else run(std::integral_constant<int, T_Q8_0>{});
    } else {
        if constexpr (TE == T_Q4_0) run(std::integral_constant<int, T_Q4_0>{});
        else run(std::integral_constant<int, T_Q8_0>{});
    }
    const int lane = tid & 63, half = lane >> 5, col = lane & 31;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int m = 8 * (i >> 2) + 4 * half + (i & 3);
        if (m < n) a.dn[(int64_t)prs[m] * a.H + r0 + wave * 32 + col] = acc[i];
    }
}

// P6: grid (ceil(H/256), T): out = sum_k fmaf(w_k, dn_k, acc) (+ shared expert)
__global__ __launch_bounds__(256) void k_pf_combine(PfArgs a) {
    const int t = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
    if (h >= a.H) return;
    float acc = 0.0f;
    for (int k = 0; k < a.K; k++)
        acc = __builtin_fmaf(a.wts[t * a.K + k], a.dn[(int64_t)(t * a.K + k) * a.H + h], acc);
    float o = acc;
    if (a.has_shared) {
        const float shv = a.dn[(int64_t)(a.T * a.K + t) * a.H + h];
        if (a.sh_gate_w) o = __builtin_fmaf(shv, 1.0f / (1.0f + det_exp(-a.glogit[t])), acc);
        else o = shv + acc;
    }
    a.out[(int64_t)t * a.H + h] = o;
}

void launch_quantize_q8_1(const float* x, void* out, int64_t ncols, int64_t ncols_padded, int64_t nrows,
                          hipStream_t s);

struct PfPlan {
    size_t logits, glogit, ids, wts, xq, off, spairs, tiles, ntiles, hq, dn, total;
    int64_t xq_stride, hq_stride;
    int max_tiles;
};

static size_t al256p(size_t n) { return (n + 255) & ~(size_t)255; }

static PfPlan plan_pf(int H, int F, int E, int K, int T) {
    PfPlan p{};
    size_t o = 0;
    const size_t P = (size_t)T * K + T;
    p.xq_stride = pad_to(H, ROW_PAD) / QK * Q8_1_BYTES;
    p.hq_stride = pad_to(F, ROW_PAD) / QK * Q8_1_BYTES;
    p.max_tiles = (int)(P / PF_TILE) + E + 2;
    p.logits = o; o += al256p((size_t)T * E * 4);
    p.glogit = o; o += al256p((size_t)T * 4);
    p.ids = o; o += al256p((size_t)T * K * 4);
    p.wts = o; o += al256p((size_t)T * K * 4);
    p.xq = o; o += al256p((size_t)T * p.xq_stride);
    p.off = o; o += al256p((size_t)(E + 2) * 4);
    p.spairs = o; o += al256p(P * 4);
    p.tiles = o; o += al256p((size_t)p.max_tiles * 3 * 4);
    p.ntiles = o; o += al256p(4);
    p.hq = o; o += al256p(P * p.hq_stride);
    p.dn = o; o += al256p(P * H * 4);
    p.total = o;
    return p;
}

template <int TE, int TS>
static void launch_pf(const PfArgs& a, const PfPlan& p, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_router, dim3(a.E + (a.sh_gate_w ? 1 : 0), (a.T + MAX_TOK - 1) / MAX_TOK), dim3(256), 0, s,
                       a);
    launch_quantize_q8_1(a.x, a.xq, a.H, p.xq_stride / Q8_1_BYTES * QK, a.T, s);
    hipLaunchKernelGGL(k_pf_topk, dim3(a.T), dim3(64), 0, s, a);
    hipLaunchKernelGGL(k_pf_plan, dim3(1), dim3(1024), 0, s, a);
    hipLaunchKernelGGL((k_pf_gate_up<TE, TS>), dim3(a.F / 64, p.max_tiles), dim3(PF_THREADS), 0, s, a);
    hipLaunchKernelGGL((k_pf_down<TE, TS>), dim3(a.H / 128, p.max_tiles), dim3(PF_THREADS), 0, s, a);
    hipLaunchKernelGGL(k_pf_combine, dim3((a.H + 255) / 256, a.T), dim3(256), 0, s, a);
}

}  // namespace chimere

using namespace chimere;

extern "C" {

size_t chimere_moe_prefill_workspace_size(const chimere_moe_layer* L, int max_ntok) {
    if (!L || max_ntok < 1) return 0;
    return plan_pf(L->hidden, L->ffn, L->n_experts, L->top_k, max_ntok).total;
}

void chimere_moe_prefill(const chimere_moe_layer* L, const float* x, float* out, int ntok, int* ids_out,
                         float* w_out, void* workspace, size_t ws_bytes, hipStream_t stream) {
    CHIMERE_REQUIRE(L && x && out && workspace, CHIMERE_ERR_ARG, "moe_prefill: null pointer");
    const int H = L->hidden, F = L->ffn, E = L->n_experts, K = L->top_k;
    CHIMERE_REQUIRE(ntok >= 1, CHIMERE_ERR_ARG, "moe_prefill: ntok=%d", ntok);
    CHIMERE_REQUIRE(H > 0 && H % 256 == 0 && F > 0 && F % 256 == 0, CHIMERE_ERR_ARG,
                    "moe_prefill: hidden=%d / ffn=%d must be multiples of 256", H, F);
    CHIMERE_REQUIRE(E >= 1 && E <= MAX_E && K >= 1 && K <= MAX_K && K <= E, CHIMERE_ERR_ARG,
                    "moe_prefill: n_experts=%d top_k=%d out of range", E, K);
    const bool has_sh = L->shared_type >= 0;
    CHIMERE_REQUIRE((L->expert_type == T_Q4_0 || L->expert_type == T_Q8_0) &&
                        (!has_sh || L->shared_type == T_Q4_0 || L->shared_type == T_Q8_0),
                    CHIMERE_ERR_ARG, "moe_prefill: Q4_0 / Q8_0 weights only (expert %d, shared %d)", L->expert_type,
                    L->shared_type);
    CHIMERE_REQUIRE(!has_sh || (L->sh_gate && L->sh_up && L->sh_down), CHIMERE_ERR_ARG,
                    "moe_prefill: shared expert incomplete");
    CHIMERE_REQUIRE(L->router_w && L->gate_exps && L->up_exps && L->down_exps, CHIMERE_ERR_ARG,
                    "moe_prefill: null weight pointer");
    CHIMERE_REQUIRE(!ids_out == !w_out, CHIMERE_ERR_ARG, "moe_prefill: ids_out and w_out go together");
    const int64_t rbH = row_bytes(L->expert_type, H), rbF = row_bytes(L->expert_type, F);
    CHIMERE_REQUIRE(L->gate_stride >= rbH * F && L->up_stride >= rbH * F && L->down_stride >= rbF * H,
                    CHIMERE_ERR_ARG, "moe_prefill: expert strides too small");
    CHIMERE_REQUIRE((((uintptr_t)L->gate_exps | (uintptr_t)L->up_exps | (uintptr_t)L->down_exps |
                      (uintptr_t)L->gate_stride | (uintptr_t)L->up_stride | (uintptr_t)L->down_stride) & 1) == 0,
                    CHIMERE_ERR_ARG, "moe_prefill: weights must be 2-byte aligned");
    const PfPlan p = plan_pf(H, F, E, K, ntok);
    CHIMERE_REQUIRE(ws_bytes >= p.total && ((uintptr_t)workspace & 255) == 0, CHIMERE_ERR_WORKSPACE,
                    "moe_prefill: workspace %zu bytes < %zu (or not 256-byte aligned)", ws_bytes, p.total);
    uint8_t* w = (uint8_t*)workspace;
    PfArgs a{};
    a.H = H; a.F = F; a.E = E; a.K = K; a.T = ntok; a.has_shared = has_sh;
    a.x = x; a.out = out; a.router = L->router_w; a.bias = L->logit_bias;
    a.gate = (const uint8_t*)L->gate_exps; a.up = (const uint8_t*)L->up_exps; a.down = (const uint8_t*)L->down_exps;
    a.sg = L->gate_stride; a.su = L->up_stride; a.sd = L->down_stride;
    a.sh_gate = (const uint8_t*)L->sh_gate; a.sh_up = (const uint8_t*)L->sh_up; a.sh_down = (const uint8_t*)L->sh_down;
    a.sh_gate_w = has_sh ? L->sh_gate_w : nullptr;
    a.ids_out = ids_out; a.w_out = w_out;
    a.logits = (float*)(w + p.logits); a.glogit = (float*)(w + p.glogit);
    a.ids = (int*)(w + p.ids); a.wts = (float*)(w + p.wts);
    a.xq = w + p.xq; a.off = (int*)(w + p.off); a.spairs = (int*)(w + p.spairs);
    a.tiles = (int*)(w + p.tiles); a.ntiles = (int*)(w + p.ntiles);
    a.hq = w + p.hq; a.dn = (float*)(w + p.dn);
    a.xq_stride = p.xq_stride; a.hq_stride = p.hq_stride; a.max_tiles = p.max_tiles;
    const int te = L->expert_type, ts = has_sh ? L->shared_type : te;
    if (te == T_Q4_0 && ts == T_Q4_0) launch_pf<T_Q4_0, T_Q4_0>(a, p, stream);
    else if (te == T_Q4_0) launch_pf<T_Q4_0, T_Q8_0>(a, p, stream);
    else if (ts == T_Q4_0) launch_pf<T_Q8_0, T_Q4_0>(a, p, stream);
    else launch_pf<T_Q8_0, T_Q8_0>(a, p, stream);
    check_launch("moe_prefill");
}

}  // extern "C"
