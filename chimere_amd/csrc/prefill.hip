// prefill.hip -- routed MoE FFN for a chunk of tokens (prefill): tokens are
// routed, grouped by expert, and each expert's gate/up and down projections
// run as int8 MFMA grouped GEMMs (v_mfma_i32_16x16x32_i8: one 32-element
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

constexpr int PF_CHUNK = 8;      // 32-element blocks per K chunk staged in LDS
constexpr int PF_TILE = 16;      // (token, k) pairs per tile: the M dimension of v_mfma_i32_16x16x32_i8
constexpr int PF_THREADS = 256;  // 4 waves
// router tile: tokens x rows per work-group (8 x 8: 100 VGPRs, four
// work-groups per CU; 16 x 8 at 170 VGPRs ran the 512-token chunk ~5 us slower)
constexpr int PF_RT = 8, PF_RE = 8;

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
    int* spairs;     // [T*K + T] pairs grouped by expert (shared expert last)
    int* tiles;      // [max_tiles][3] (expert, start, count)
    int* ntiles;     // [1]
    uint8_t* hq;     // [T*K + T][hq_stride] Q8_1(h) per pair
    float* dn;       // [T*K + T][H] down-projection output per pair
    // per-block metadata of xq / hq (row strides xq_stride / 36, hq_stride /
    // 36 entries): f32 of the stored f16 scale, and -8 * (sum of the quants)
    float* xmd;
    int* xms;
    float* hmd;
    int* hms;
    int64_t xq_stride, hq_stride;
    int max_tiles;
};

// P1: grid (ceil((E + has_gate) / PF_RE), ceil(T / PF_RT)), 256 threads: logits
// of PF_RT tokens x PF_RE router rows.  Every output keeps the reference's order
// (elementwise.rs:186-221 launched with 256 threads): thread j accumulates
// columns j, j+256, ... with fma, then the 256 partials are summed by the
// halving tree (pairs j, j+m for m = 128, ..., 1).  Thread j owns partial j
// of all PF_RT * PF_RE outputs of the tile; the tree runs in LDS for 32 outputs at a
// time: 8 threads per output, thread q first reduces the 32 partials
// j = q (mod 8) (tree levels m = 128 .. 8), then levels 4, 2, 1 run across
// the 8 lanes.
__global__ __launch_bounds__(256) void k_pf_router(PfArgs a) {
    __shared__ float red[32][264];   // row stride = 8 banks: the 8-lane groups read distinct banks
    const int tid = threadIdx.x;
    const int NR = a.E + (a.sh_gate_w ? 1 : 0);
    // 1-D grid of ET x TT tiles.  Work-groups are dealt to the 8 XCDs
    // round-robin; when TT is a multiple of 8, XCD x takes the token tiles
    // [x TT/8, (x+1) TT/8) against every router row, so each XCD's L2 holds
    // the router once and only its own tokens' rows
    const int ET = (NR + PF_RE - 1) / PF_RE, TT = (a.T + PF_RT - 1) / PF_RT;
    int et, tt;
    if ((TT & 7) == 0) {
        const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
        tt = x * (TT >> 3) + k / ET;
        et = k - (k / ET) * ET;
    } else {
        tt = blockIdx.x / ET;
        et = blockIdx.x - tt * ET;
    }
    const int e0 = et * PF_RE, t0 = tt * PF_RT;
    const float* rows[PF_RE];
#pragma unroll
    for (int e = 0; e < PF_RE; e++) {
        const int r = min(e0 + e, NR - 1);
        rows[e] = r < a.E ? a.router + (int64_t)r * a.H : a.sh_gate_w;
    }
    float acc[PF_RT][PF_RE];
    // the loads of column step h + 256 are issued before step h's products;
    // the loop runs two column steps per trip on two register sets (no
    // copies between the sets), and every load is a uniform row base plus a
    // 32-bit lane offset (no 64-bit address arithmetic per load)
    const float* xr[PF_RT];
#pragma unroll
    for (int t = 0; t < PF_RT; t++) xr[t] = a.x + (int64_t)min(t0 + t, a.T - 1) * a.H;
    auto ld = [](const float* base, int h) {
        return *(const float*)((const char*)base + (uint32_t)h * 4u);
    };
    float r0[PF_RE], x0[PF_RT], r1[PF_RE], x1[PF_RT];
    auto load = [&](float (&r)[PF_RE], float (&x)[PF_RT], int h) {
#pragma unroll
        for (int e = 0; e < PF_RE; e++) r[e] = ld(rows[e], h);
#pragma unroll
        for (int t = 0; t < PF_RT; t++) x[t] = ld(xr[t], h);
    };
    auto step = [&](const float (&r)[PF_RE], const float (&x)[PF_RT]) {
#pragma unroll
        for (int t = 0; t < PF_RT; t++)
#pragma unroll
            for (int e = 0; e < PF_RE; e++) acc[t][e] = __builtin_fmaf(r[e], x[t], acc[t][e]);
    };
    // column step tid (acc = fmaf(r, x, 0), the first fma of the chain)
    load(r0, x0, tid);
    load(r1, x1, tid + 256 < a.H ? tid + 256 : tid);
#pragma unroll
    for (int t = 0; t < PF_RT; t++)
#pragma unroll
        for (int e = 0; e < PF_RE; e++) acc[t][e] = __builtin_fmaf(r0[e], x0[t], 0.0f);
    // h: the step whose operands are in set 1 (H is a multiple of 256, so
    // every bound below is uniform)
    for (int h = tid + 256; h < a.H; h += 512) {
        load(r0, x0, h + 256 < a.H ? h + 256 : h);
        step(r1, x1);
        if (h + 256 >= a.H) break;
        load(r1, x1, h + 512 < a.H ? h + 512 : h);
        step(r0, x0);
    }
    const int o = tid >> 3, q = tid & 7;
#pragma unroll
    for (int rnd = 0; rnd < PF_RT * PF_RE / 32; rnd++) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int oo = rnd * 32 + i;
            red[i][tid] = acc[oo / PF_RE][oo % PF_RE];
        }
        __syncthreads();
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = red[o][q + 8 * i];
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1)
#pragma unroll
            for (int i = 0; i < m; i++) v[i] = v[i] + v[i + m];
        float w = v[0];
        w = w + xlane<4>(w);
        w = w + xlane<2>(w);
        w = w + xlane<1>(w);
        const int oo = rnd * 32 + o, t = t0 + oo / PF_RE, e = e0 + oo % PF_RE;
        if (q == 0 && t < a.T && e < NR) {
            if (e < a.E) a.logits[(int64_t)t * a.E + e] = a.bias ? w + a.bias[e] : w;
            else a.glogit[t] = w;
        }
    }
}

// P2: one wave per token
__global__ __launch_bounds__(64) void k_pf_topk(PfArgs a) {
    __shared__ uint64_t s_tk[128];
    const int t = blockIdx.x;
    // the token's Q8_1 block metadata for the gate/up launch (f32 of the
    // stored scale, -8 * quant sum), while the logits load
    const int64_t nbx = a.xq_stride / Q8_1_BYTES;
    for (int b = threadIdx.x; b < a.H / QK; b += 64) {
        const uint8_t* blk = a.xq + (int64_t)t * a.xq_stride + (int64_t)b * Q8_1_BYTES;
        int sq = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) sq = dot4(*(const int*)(blk + 4 + 4 * k), 0x01010101, sq);
        a.xmd[t * nbx + b] = h2f(*(const uint16_t*)blk);
        a.xms[t * nbx + b] = -8 * sq;
    }
    topk_wave_any(a.logits + (int64_t)t * a.E, a.E, a.K, a.ids + t * a.K, a.wts + t * a.K, s_tk);
}

// exclusive prefix sum of one int per thread over a 1024-thread group
__device__ __forceinline__ int excl_scan1024(int v, int* wsum, int* total) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    if (w == 0) {
        const int t = lane < 16 ? wsum[lane] : 0;
        int sc = t;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const int y = __shfl_up(sc, d);
            if (lane >= d) sc += y;
        }
        __syncthreads();   // pairs with the barrier below for the other waves
        if (lane < 16) wsum[lane] = sc - t;
        if (lane == 15) *total = sc;
    } else {
        __syncthreads();
    }
    __syncthreads();
    return x - v + wsum[w];
}

// P3: one 1024-thread work-group.  Counting sort of the T*K pairs by expert
// (the order of pairs inside an expert does not affect any result: every
// pair's output row is computed on its own), the shared expert as expert E
// with all T tokens, and the list of 16-pair tiles.  Thread i owns experts
// 2i and 2i+1 in the scans.
__global__ __launch_bounds__(1024) void k_pf_plan(PfArgs a) {
    __shared__ int cnt[2 * 1024], fill[MAX_E + 1];
    __shared__ int wsum[16], tot[2];
    const int tid = threadIdx.x, TK = a.T * a.K, NE = a.E + 1;
    for (int e = tid; e < 2 * 1024; e += 1024) cnt[e] = 0;
    for (int e = tid; e < NE; e += 1024) fill[e] = 0;
    __syncthreads();
    // pairs in batches of 4 per thread: the 4 id loads (and weight loads)
    // are issued together (one memory round trip per batch, not per pair);
    // the first batch's ids and weights stay in registers for the scatter
    int k4[4];
    float kw[4];
    for (int p0 = tid; p0 < TK; p0 += 4 * 1024) {
        int e4[4];
        float w4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const bool in = p0 + i * 1024 < TK;
            e4[i] = in ? a.ids[p0 + i * 1024] : -1;
            w4[i] = in && a.ids_out ? a.wts[p0 + i * 1024] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (e4[i] >= 0) atomicAdd(&cnt[e4[i]], 1);
        if (p0 == tid) {
#pragma unroll
            for (int i = 0; i < 4; i++) { k4[i] = e4[i]; kw[i] = w4[i]; }
        }
    }
    if (tid == 0) cnt[a.E] = a.has_shared ? a.T : 0;
    __syncthreads();
    const int c0 = cnt[2 * tid], c1 = cnt[2 * tid + 1];
    const int n0 = (c0 + PF_TILE - 1) / PF_TILE, n1 = (c1 + PF_TILE - 1) / PF_TILE;
    const int po = excl_scan1024(c0 + c1, wsum, &tot[0]);
    const int to = excl_scan1024(n0 + n1, wsum, &tot[1]);
    __syncthreads();
    cnt[2 * tid] = po;                 // cnt now holds each expert's first position
    cnt[2 * tid + 1] = po + c0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int e = 2 * tid + h, c = h ? c1 : c0, base = h ? po + c0 : po, tb = h ? to + n0 : to;
        for (int s = 0; s * PF_TILE < c; s++) {
            a.tiles[(tb + s) * 3] = e;
            a.tiles[(tb + s) * 3 + 1] = base + s * PF_TILE;
            a.tiles[(tb + s) * 3 + 2] = min(PF_TILE, c - s * PF_TILE);
        }
    }
    if (tid == 0) *a.ntiles = tot[1];
    __syncthreads();
    for (int p0 = tid; p0 < TK; p0 += 4 * 1024) {
        int e4[4];
        float w4[4];
        if (p0 == tid) {
#pragma unroll
            for (int i = 0; i < 4; i++) { e4[i] = k4[i]; w4[i] = kw[i]; }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bool in = p0 + i * 1024 < TK;
                e4[i] = in ? a.ids[p0 + i * 1024] : -1;
                w4[i] = in && a.ids_out ? a.wts[p0 + i * 1024] : 0.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = p0 + i * 1024, e = e4[i];
            if (e < 0) continue;
            a.spairs[cnt[e] + atomicAdd(&fill[e], 1)] = p;
            if (a.ids_out) { a.ids_out[p] = e; a.w_out[p] = w4[i]; }
        }
    }
    if (a.has_shared)
        for (int t = tid; t < a.T; t += 1024) a.spairs[cnt[a.E] + t] = TK + t;
}

// ---- grouped GEMM on v_mfma_i32_16x16x32_i8.  Layout: lane l supplies row
// l%16 of A and column l%16 of B, elements 8*(l/16) .. +8 of the K = 32
// block; result D[i] at lane l is (row 4*(l/16) + i, column l%16).  A = the
// tile's 16 Q8_1 activation rows (pairs), B = 16 weight rows; one 32-element
// quantization block per instruction, so each result is the exact int32
// block dot.  Q4_0 enters as the unsigned nibbles and the accumulator starts
// at -8 * sum(q_x) of the pair's block, which makes the result
// sum((nib - 8) * q_x).

// bytes of a PF_CHUNK-block chunk of a row (IQ3_S: one 110-byte superblock)
template <int T>
constexpr int pf_row_chunk_bytes() {
    return QTraits<T>::ELEMS == 256 ? PF_CHUNK / 8 * QTraits<T>::BYTES : PF_CHUNK * QTraits<T>::BYTES;
}

// LDS row stride of a staged chunk on the two-stage path: the chunk bytes,
// or for IQ3_S / Q6_K the 16-byte aligned span that holds the superblock (it
// starts at (110 c) % 16 / (210 c) % 16 inside the span: at most 14 + 110 /
// 14 + 210 bytes)
template <int T>
constexpr int pf_lds_row() { return T == T_IQ3_S ? 128 : T == T_Q6_K ? 224 : pf_row_chunk_bytes<T>(); }

// LDS row strides of the two-stage path, padded so that the 16 rows a wave
// reads at one block offset spread over the banks: a stride that is a
// multiple of 128 bytes puts every row on the same banks (IQ3_S: 128 -> 144);
// the activation rows (PF_CHUNK Q8_1 blocks, 288 bytes) get one more 16-byte
// piece (304: the A-fragment reads of a half-wave on distinct banks)
template <int T>
constexpr int pf_lds_row_al() { return pf_lds_row<T>() % 128 == 0 ? pf_lds_row<T>() + 16 : pf_lds_row<T>(); }
constexpr int PF_XROW = PF_CHUNK * 36, PF_XROW_AL = PF_XROW + 16;

__constant__ uint32_t c_iq3s_grid_pf[512] = CHIMERE_IQ3S_GRID_INIT;

// 8 weight values of block b of an LDS row as int8, and f32(d); IQ3_S also
// sets *mult = 1 + 2 * (4-bit scale of sub-block b), the factor of its exact
// block dot (cs/src/kernels/iq3s_gemv.rs:292-352)
// Per-superblock fields of an IQ3_S chunk row (read once per chunk): f16 d,
// the 8 qh bytes, the 4 scale bytes
struct PfSb {
    uint32_t d, qh0, qh1, sc;
};
template <int T>
__device__ __forceinline__ void pf_sb(const uint8_t* row, PfSb& f) {
    if constexpr (T == T_IQ3_S) {
        f.d = lds_u16(row, 0);
        f.qh0 = lds_u32(row, 66);
        f.qh1 = lds_u32(row, 70);
        f.sc = lds_u32(row, 106);
    }
}

template <int T>
constexpr bool pf_kq() { return T == T_Q4_K || T == T_Q5_K; }

// K-quant superblock fields of block b (Q4_K / Q5_K, 4-byte aligned LDS row):
// f32(dmin) and the 6-bit min m of sub-block b (gguf_loader.rs:1150-1163)
struct PfMin {
    float dm;
    int m;
};

template <int T, bool PRE>
__device__ __forceinline__ long pf_b_frag(const uint8_t* row, int b, int q, uint32_t* dw, int* mult,
                                          const uint32_t* grid, const PfSb& f, PfMin* mn = nullptr) {
    uint32_t lo, hi;
    if constexpr (pf_kq<T>()) {
        // sub-block b of the superblock [f16 d][f16 dmin][scales 12]([qh 32])[qs 128]:
        // lane group q holds elements 8q .. 8q+7 = nibble (b & 1) of qs[32 (b/2) + l]
        // (Q5_K: plus bit b of qh[l] as bit 4), unsigned; the MFMA gives
        // sum q * q_x, the scale multiplies it and the min term is added apart
        const uint32_t* u = (const uint32_t*)row;
        const uint32_t w0 = u[0];
        *dw = w0 & 0xFFFFu;
        int sc, m;
        kq_scale_min(u[1], u[2], u[3], b, sc, m);
        *mult = sc;
        mn->dm = h2f(w0 >> 16);
        mn->m = m;
        constexpr int QS = T == T_Q5_K ? 48 : 16;
        const uint32_t* qs = (const uint32_t*)(row + QS + 32 * (b >> 1) + 8 * q);
        const int sh = 4 * (b & 1);
        lo = (qs[0] >> sh) & 0x0F0F0F0Fu;
        hi = (qs[1] >> sh) & 0x0F0F0F0Fu;
        if constexpr (T == T_Q5_K) {
            const uint32_t* qh = (const uint32_t*)(row + 16 + 8 * q);
            lo |= ((qh[0] >> b) & 0x01010101u) << 4;
            hi |= ((qh[1] >> b) & 0x01010101u) << 4;
        }
    } else if constexpr (T == T_Q6_K) {
        // block b = 4 gi + jj of the superblock [ql 128][qh 64][scales 16 x i8][f16 d]
        // (gguf_loader.rs:839-917): element l of the block is nibble jj / 2 of
        // ql[64 gi + 32 (jj & 1) + l] with bits 2 jj, 2 jj + 1 of qh[32 gi + l]
        // as bits 4, 5, minus 32; lane group q holds elements 8q .. 8q+7.  The
        // block's two 16-element halves have their own int8 scales: *mult holds
        // both (low byte: elements 0..15, high byte: 16..31)
        const int gi = b >> 2, jj = b & 3;
        const int lo_off = 64 * gi + 32 * (jj & 1) + 8 * q, hi_off = 128 + 32 * gi + 8 * q;
        const int nsh = 4 * (jj >> 1), hsh = 2 * jj;
        uint32_t v[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t u = ((lds_u32(row, lo_off + 4 * i) >> nsh) & 0x0F0F0F0Fu) |
                               (((lds_u32(row, hi_off + 4 * i) >> hsh) & 0x03030303u) << 4);
            const uint32_t t = u ^ 0x20202020u, sgn = t & 0x20202020u;   // u - 32 per byte, 6-bit
            v[i] = t | (sgn << 1) | (sgn << 2);                             // sign-extended
        }
        lo = v[0];
        hi = v[1];
        *dw = lds_u16(row, 208);
        *mult = (int)lds_u16(row, 192 + 8 * gi + 2 * jj);
    } else if constexpr (T == T_IQ3_S) {
        // sub-block b of the superblock [f16 d][qs 64][qh 8][signs 32][scales 4];
        // lane group q holds elements 8q .. 8q+7: grid entries qs[8b+2q] and
        // qs[8b+2q+1] with high bits 2q and 2q+1 of qh[b], negated per byte by
        // bits 0..3 / 4..7 of signs[4b+q]
        *dw = PRE ? f.d : lds_u16(row, 0);
        const uint32_t qs = lds_u16(row, 2 + 8 * b + 2 * q);
        uint32_t i0, i1;
        if constexpr (PRE) {
            // high bits 2q, 2q+1 of the superblock's qh bytes as 0/1 bytes
            // (formed once per superblock: the same for every block), each
            // index one v_perm: byte 0 from qs, byte 1 the block's high bit
            const uint32_t w = b < 4 ? f.qh0 : f.qh1;
            const uint32_t h0 = (w >> (2 * q)) & 0x01010101u, h1 = (w >> (2 * q + 1)) & 0x01010101u;
            const uint32_t sel = 0x0C0C0000u | ((uint32_t)(4 + (b & 3)) << 8);
            i0 = __builtin_amdgcn_perm(h0, qs, sel);
            i1 = __builtin_amdgcn_perm(h1, qs, sel | 1u);
        } else {
            const uint32_t qh = (uint32_t)row[66 + b] >> (2 * q);
            i0 = (qs & 0xFFu) | ((qh & 1u) << 8);
            i1 = (qs >> 8) | ((qh & 2u) << 7);
        }
        const uint32_t sg = row[74 + 4 * b + q];
        // byte masks of the two sign nibbles, negation as (g ^ m) + (m & 1)
        // per byte
        uint32_t m0, m1;
        byte_sign_masks(sg, 0, m0, m1);
        lo = (grid[i0] ^ m0) + (m0 & 0x01010101u);
        hi = (grid[i1] ^ m1) + (m1 & 0x01010101u);
        *mult = 1 + 2 * (int)(((PRE ? f.sc >> (4 * b) : row[106 + (b >> 1)] >> (4 * (b & 1)))) & 0xFu);
    } else if constexpr (T == T_Q4_0) {
        // bytes o .. o+7 of the row hold the 16 nibbles (low nibbles for
        // q < 2, high for q >= 2); o is 2 mod 4 for even b, 0 mod 4 for odd
        // b, so three aligned dwords and one funnel shift per result dword
        // (byte alignment and nibble select in one) do it
        const int off = b * 18;
        *dw = lds_u16(row, off);
        const int o = off + 2 + 8 * (q & 1), a = o & ~3, sh = 8 * (o & 3) + 4 * (q >> 1);
        const uint32_t* w = (const uint32_t*)(row + a);
        const uint32_t d0 = w[0], d1 = w[1], d2 = w[2];
        lo = __builtin_amdgcn_alignbit(d1, d0, sh) & 0x0F0F0F0Fu;
        hi = __builtin_amdgcn_alignbit(d2, d1, sh) & 0x0F0F0F0Fu;
    } else {
        const int off = b * 34;
        *dw = lds_u16(row, off);
        lo = lds_u32(row, off + 2 + 8 * q);
        hi = lds_u32(row, off + 6 + 8 * q);
    }
    (void)mult;
    (void)grid;
    (void)f;
    (void)mn;
    return (long)(((uint64_t)hi << 32) | lo);
}

// Per-block metadata of the staged activation blocks (PF_TILE pairs x
// PF_CHUNK blocks, pair-major, 36 bytes each): xd[b][m] = f32(d),
// xs8[b][m] = -8 * sum(q) (Q4_0 correction; the MFMA accumulator's start)
__device__ __forceinline__ void pf_xmeta(const uint8_t* xl, float* xd, int* xs8, int xr) {
    const int i = threadIdx.x;
    if (i < PF_TILE * PF_CHUNK) {
        const int m = i / PF_CHUNK, b = i % PF_CHUNK;
        const uint8_t* blk = xl + m * xr + b * 36;
        int s = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) s = dot4(*(const int*)(blk + 4 + 4 * k), 0x01010101, s);
        xs8[b * PF_TILE + m] = -8 * s;
        xd[b * PF_TILE + m] = h2f(*(const uint16_t*)blk);
    }
}

// Issues (asynchronously) one K chunk: `nrows` weight rows of `cbytes`
// bytes (global stride rb) and the tile's PF_TILE activation rows (row
// xrows[m] of src, stride xstride, chunk at byte xoff).
__device__ __forceinline__ void pf_issue(uint8_t* wl, const uint8_t* w, int64_t rb, int nrows, int cbytes,
                                         uint8_t* xl, const uint8_t* xsrc, const int* xrows, int64_t xstride,
                                         int64_t xoff) {
    stage_rows(wl, w, rb, nrows, cbytes, threadIdx.x, PF_THREADS);
    constexpr int PER = 36 * PF_CHUNK / 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int c0 = wave * 64; c0 < PF_TILE * PER; c0 += PF_THREADS) {
        const int c = c0 + lane;
        if (c < PF_TILE * PER) {
            const int r = c / PER, col = c - r * PER;
            __builtin_amdgcn_global_load_lds((const glb_void_t*)(xsrc + xrows[r] * xstride + xoff + col * 16),
                                             (lds_void_t*)(xl + c0 * 16), 16, 0, 0);
        }
    }
}

// One staged K chunk for a wave's NTN 16-row column tiles (weight rows
// wrows + 16*n, LDS row stride cbytes): acc[n][i] = output (pair 4*(l/16)+i,
// row 16n + l%16), updated per block as fmaf(f32(d_w)*f32(d_x), sumi, acc).
// PRE: read the per-superblock fields of the rows once per chunk (measured
// faster on the two-stage gate/up path, slower on the one-stage down path)
template <int T, int NTN, bool PRE>
__device__ __forceinline__ void pf_mma_chunk(const uint8_t* xl, int xr, const float* xd, const int* xs8,
                                             const uint8_t* wrows, int cbytes, int nb, const uint32_t* grid,
                                             float (&acc)[NTN][4]) {
    const int lane = threadIdx.x & 63, q = lane >> 4, c = lane & 15;
    // two blocks in flight: block b's matrix products are issued before block
    // b-1's results are rescaled, so the MFMA latency overlaps VALU work
    v4i r[NTN], rp[NTN];
    v4i r2[NTN], rp2[NTN];     // Q6_K: the products of the block's second 16-element half
    float dw[NTN], dwp[NTN];
    int mu[NTN], mup[NTN];   // IQ3_S / K-quant sub-block factors
    PfMin mn[NTN], mnp[NTN];   // K-quant min terms
    int4 sqp;                  // K-quant: sum of the pairs' quants of the previous block
    PfSb sb[NTN];
#pragma unroll
    for (int n = 0; n < NTN; n++)
        if constexpr (PRE) pf_sb<T>(wrows + (16 * n + c) * cbytes, sb[n]);
    float4 dxp;
    for (int b = 0; b <= nb; b++) {
        float4 dx;
        if (b < nb) {
            const uint8_t* ab = xl + c * xr + b * 36 + 4 + 8 * q;
            const long af = (long)(((uint64_t) * (const uint32_t*)(ab + 4) << 32) | *(const uint32_t*)ab);
            dx = *(const float4*)(xd + b * PF_TILE + 4 * q);
            v4i c0 = {0, 0, 0, 0};
            if constexpr (T == T_Q4_0) c0 = *(const v4i*)(xs8 + b * PF_TILE + 4 * q);
#pragma unroll
            for (int n = 0; n < NTN; n++) {
                uint32_t dwb;
                const long bf =
                    pf_b_frag<T, PRE>(wrows + (16 * n + c) * cbytes, b, q, &dwb, &mu[n], grid, sb[n], &mn[n]);
                dw[n] = h2f(dwb);
                if constexpr (T == T_Q6_K) {
                    // the two halves (lane groups 0, 1 and 2, 3) in separate
                    // products, each scaled by its own factor below
                    r[n] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, q < 2 ? bf : 0l, c0, 0, 0, 0);
                    r2[n] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, q < 2 ? 0l : bf, c0, 0, 0, 0);
                } else {
                    r[n] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, c0, 0, 0, 0);
                }
            }
        }
        if (b > 0) {
            if constexpr (T == T_IQ3_S || pf_kq<T>()) {
#pragma unroll
                for (int n = 0; n < NTN; n++)
#pragma unroll
                    for (int i = 0; i < 4; i++) rp[n][i] = __mul24(rp[n][i], mup[n]);   // |.| < 2^21
            }
            if constexpr (T == T_Q6_K) {
                // the exact block dot lo * sc0 + hi * sc1 (|.| <= 2 * 16*32*127*128 < 2^24)
#pragma unroll
                for (int n = 0; n < NTN; n++) {
                    const int s0 = (int)(int8_t)(mup[n] & 0xFF), s1 = (int)(int8_t)((mup[n] >> 8) & 0xFF);
#pragma unroll
                    for (int i = 0; i < 4; i++) rp[n][i] = __mul24(rp[n][i], s0) + __mul24(rp2[n][i], s1);
                }
            }
#pragma unroll
            for (int n = 0; n < NTN; n++) {
                acc[n][0] = __builtin_fmaf(dwp[n] * dxp.x, (float)rp[n][0], acc[n][0]);
                acc[n][1] = __builtin_fmaf(dwp[n] * dxp.y, (float)rp[n][1], acc[n][1]);
                acc[n][2] = __builtin_fmaf(dwp[n] * dxp.z, (float)rp[n][2], acc[n][2]);
                acc[n][3] = __builtin_fmaf(dwp[n] * dxp.w, (float)rp[n][3], acc[n][3]);
                if constexpr (pf_kq<T>()) {
                    // the min term of the block: fmaf(-(f32(dmin) * f32(d_x)), (float)(m * sum q_x), acc)
                    acc[n][0] = __builtin_fmaf(-(mnp[n].dm * dxp.x), (float)__mul24(mnp[n].m, sqp.x), acc[n][0]);
                    acc[n][1] = __builtin_fmaf(-(mnp[n].dm * dxp.y), (float)__mul24(mnp[n].m, sqp.y), acc[n][1]);
                    acc[n][2] = __builtin_fmaf(-(mnp[n].dm * dxp.z), (float)__mul24(mnp[n].m, sqp.z), acc[n][2]);
                    acc[n][3] = __builtin_fmaf(-(mnp[n].dm * dxp.w), (float)__mul24(mnp[n].m, sqp.w), acc[n][3]);
                }
                // the block's rescale stays in its iteration: without this the
                // fmas of the unrolled blocks sink below all of their matrix
                // products, which then hold 36 more registers
                asm volatile("" : "+v"(acc[n][0]), "+v"(acc[n][1]), "+v"(acc[n][2]), "+v"(acc[n][3]));
            }
        }
#pragma unroll
        for (int n = 0; n < NTN; n++) { rp[n] = r[n]; rp2[n] = r2[n]; dwp[n] = dw[n]; mup[n] = mu[n]; mnp[n] = mn[n]; }
        dxp = dx;
        // nor do the scheduler's clusters of matrix products span blocks
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (pf_kq<T>()) {
            // sum q_x = -(xs8 / 8) of the block just issued (xs8 = -8 * sum q_x)
            if (b < nb) {
                const int4 s8 = *(const int4*)(xs8 + b * PF_TILE + 4 * q);
                sqp = make_int4(-(s8.x >> 3), -(s8.y >> 3), -(s8.z >> 3), -(s8.w >> 3));
            }
        }
    }
}

// LDS buffers of one pipeline stage: the weight chunk rows, the tile's
// activation chunk and its per-block metadata
struct PfStage {
    uint8_t* w;
    uint8_t* x;
    float* xd;
    int* xs;
};

// K loop of one work-group: NR weight rows (n0 at w0, the rest at w1; global
// row stride rb), activation rows xrows of xsrc; wave `wave` computes NTN
// 16-row tiles at LDS row wrow0.
//
// With 16-byte aligned rows: two stages, chunk c + 1 copied into one while
// chunk c is computed from the other.  Every copy of a chunk (weight rows and
// activation rows) is one untracked 16-byte copy per lane from a single loop,
// so the compiler adds no waits of its own (its alias analysis does not
// separate the stages), and the barriers wait for LDS accesses only: the
// release fence of __syncthreads() would also wait for the copies in flight.
// Otherwise one stage, copied and waited for per chunk.
// SPAN: the one-stage path's dword span copies (below) for 4-byte aligned rows
template <int T, int NTN, int NR, bool AL, bool SPAN = false>
__device__ __forceinline__ void pf_gemm_k(const PfStage& s0, const PfStage& s1, const uint8_t* w0, int n0,
                                          const uint8_t* w1, int64_t rb, int nbk, const uint8_t* xsrc,
                                          const int* xrows, int64_t xstride, const float* xmd, const int* xms,
                                          int wrow0, const uint32_t* grid, float (&acc)[NTN][4]) {
    constexpr int CB = pf_row_chunk_bytes<T>(), CBL = pf_lds_row<T>(), CBLP = pf_lds_row_al<T>();
    static_assert(!AL || (CBL % 16 == 0 && CBLP % 16 == 0), "chunk rows in 16-byte pieces");
    // pieces per row (copied) and per LDS row slot (the rest of a slot is padding)
    constexpr int PCB = CBL / 16, PCBP = CBLP / 16, PER = PF_XROW / 16, PERP = PF_XROW_AL / 16;
    constexpr int TW = NR * PCBP, TWP = (TW + 63) & ~63, TOT = TWP + PF_TILE * PERP;
#pragma unroll
    for (int n = 0; n < NTN; n++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[n][i] = 0.0f;
    const int nc = nbk / PF_CHUNK;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (!AL) {
        // SPAN and 4-byte aligned rows (IQ3_S rows of 2 superblocks, Q6_K ...):
        // chunk c is copied as the dword-aligned span holding it, `pre` bytes
        // into LDS rows of stride CBLP, with dword asynchronous copies mapped
        // piece -> (row, column) by constant divisors; other rows go through
        // stage_rows
        constexpr int LP = CBLP / 4, NW = PF_THREADS / 64;   // the padded row stride (banks)
        const bool al4 = (((uintptr_t)w0 | (uintptr_t)w1 | (uintptr_t)rb) & 3) == 0;
        // IQ3_S rows (even addresses; the decode reads bytes and halfwords
        // only), one 16-row tile per wave: each row's chunk is copied as the
        // 16-byte aligned span holding it, starting (row address + chunk
        // offset) % 16 bytes into its LDS row -- per lane, since lane c reads
        // row c of the tile.  An aligned 16-byte piece never leaves the page
        // of the valid bytes it holds.
        constexpr bool S16 = SPAN && T == T_IQ3_S && NTN == 1;
        static_assert(!S16 || ((CB + 15 + 15) / 16 * 16 <= CBLP && CBLP % 16 == 0), "IQ3_S span fits its row");
        for (int c = 0; c < nc; c++) {
            const int64_t goff = (int64_t)c * CB, xoff = (int64_t)c * PF_CHUNK * 36;
            const int pre = (int)(goff & 3);
            const bool span = SPAN && al4 && pre + CB <= CBLP;
            if (S16 && span) {
                constexpr int LQ = CBLP / 16;   // 16-byte slots per LDS row
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const uintptr_t b1 = (uintptr_t)(w0 + goff);
                const uintptr_t b2 = (uintptr_t)(w1 + goff) - (uintptr_t)((int64_t)n0 * rb);
#pragma unroll
                for (int k = 0; k < (NR * LQ + PF_THREADS - 1) / PF_THREADS; k++) {
                    const int c0 = (k * NW + wave) * 64;
                    const unsigned cc = (unsigned)(c0 + ln), r = cc / LQ, col = cc - r * LQ;
                    if (cc < (unsigned)(NR * LQ)) {
                        const uintptr_t ra = ((int)r < n0 ? b1 : b2) + (uintptr_t)((int64_t)r * rb);
                        const uintptr_t st = ra & ~(uintptr_t)15;
                        if ((uintptr_t)col * 16 < ra + CB - st)
                            __builtin_amdgcn_global_load_lds((const glb_void_t*)(st + col * 16),
                                                             (lds_void_t*)(s0.w + c0 * 16), 16, 0, 0);
                    }
                }
                pf_issue(nullptr, nullptr, rb, 0, CB, s0.x, xsrc, xrows, xstride, xoff);
            } else if (span) {
                const int sp = (pre + CB + 3) >> 2;   // dwords per row (the span ends inside the row)
                // the lane through an empty asm: the piece addresses are formed
                // here, not hoisted (registers) out of the chunk loop
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const uintptr_t b1 = (uintptr_t)(w0 + goff - pre);
                const uintptr_t b2 = (uintptr_t)(w1 + goff - pre) - (uintptr_t)((int64_t)n0 * rb);
#pragma unroll
                for (int k = 0; k < (NR * LP + PF_THREADS - 1) / PF_THREADS; k++) {
                    const int c0 = (k * NW + wave) * 64;
                    const unsigned cc = (unsigned)(c0 + ln), r = cc / LP, col = cc - r * LP;
                    if (cc < (unsigned)(NR * LP) && (int)col < sp) {
                        const uint8_t* src = (const uint8_t*)(((int)r < n0 ? b1 : b2) + (uintptr_t)((int64_t)r * rb) +
                                                              col * 4);
                        __builtin_amdgcn_global_load_lds((const glb_void_t*)src, (lds_void_t*)(s0.w + c0 * 4), 4, 0,
                                                         0);
                    }
                }
                pf_issue(nullptr, nullptr, rb, 0, CB, s0.x, xsrc, xrows, xstride, xoff);
            } else {
                stage_rows(s0.w, w0 + goff, rb, n0, CB, threadIdx.x, PF_THREADS);
                pf_issue(s0.w + n0 * CB, w1 + goff, rb, NR - n0, CB, s0.x, xsrc, xrows, xstride, xoff);
            }
            lds_copy_wait();
            __syncthreads();
            pf_xmeta(s0.x, s0.xd, s0.xs, PF_XROW);
            __syncthreads();
            if (S16 && span) {
                const int rl = wrow0 + (lane & 15);   // this lane's row
                const uintptr_t ra = (rl < n0 ? (uintptr_t)w0 + (uintptr_t)((int64_t)rl * rb)
                                              : (uintptr_t)w1 + (uintptr_t)((int64_t)(rl - n0) * rb)) +
                                     (uintptr_t)goff;
                pf_mma_chunk<T, NTN, false>(s0.x, PF_XROW, s0.xd, s0.xs, s0.w + wrow0 * CBLP + (int)(ra & 15), CBLP,
                                            PF_CHUNK, grid, acc);
            } else if (span)
                pf_mma_chunk<T, NTN, false>(s0.x, PF_XROW, s0.xd, s0.xs, s0.w + wrow0 * CBLP + pre, CBLP, PF_CHUNK,
                                            grid, acc);
            else
                pf_mma_chunk<T, NTN, false>(s0.x, PF_XROW, s0.xd, s0.xs, s0.w + wrow0 * CB, CB, PF_CHUNK, grid, acc);
            __syncthreads();
        }
    } else {
        // Each thread copies the same pieces of every chunk (piece cc of the
        // loop below: weight row cc / PCB, column cc % PCB, or activation row
        // r, column col): their source addresses are formed once here and a
        // chunk only adds its byte offset.
        constexpr int NIT = (TOT + PF_THREADS - 1) / PF_THREADS;
        const uint8_t* psrc[NIT];
        bool pval[NIT];
        int pcol[NIT];   // column byte of a weight piece (used by the span clamp)
#pragma unroll
        for (int k = 0; k < NIT; k++) {
            const int c0 = wave * 64 + k * PF_THREADS, cc = c0 + lane;
            psrc[k] = nullptr;
            pval[k] = false;
            pcol[k] = 0;
            if (c0 < TWP) {
                if (cc < TW) {
                    const int row = cc / PCBP, col = cc - row * PCBP;
                    if (col < PCB) {
                        psrc[k] = (row < n0 ? w0 + row * rb : w1 + (row - n0) * rb) + col * 16;
                        pcol[k] = col * 16;
                        pval[k] = true;
                    }
                }
            } else if (c0 < TOT) {
                const int xc = cc - TWP;
                if (xc < PF_TILE * PERP) {
                    const int r = xc / PERP, col = xc - r * PERP;
                    if (col < PER) {
                        psrc[k] = xsrc + xrows[r] * xstride + col * 16;
                        pval[k] = true;
                    }
                }
            }
        }
        // the chunk's activation metadata (xd, xs of the stage: entry
        // b * PF_TILE + m for block b of row m) from the precomputed arrays:
        // waves 0, 1 the scales, waves 2, 3 the sums, one dword copy each
        static_assert(PF_THREADS == 256 && PF_TILE * PF_CHUNK == 128, "metadata copy geometry");
        const int64_t mstride = xstride / 36;
        const int me = (wave & 1) * 64 + lane, mb = me / PF_TILE, mm = me - mb * PF_TILE;
        const void* msrc = wave < 2 ? (const void*)(xmd + xrows[mm] * mstride + mb)
                                    : (const void*)(xms + xrows[mm] * mstride + mb);
        auto issue = [&](int c, const PfStage& s) {
            const int64_t goff = (int64_t)c * CB & ~(int64_t)15, xoff = (int64_t)c * PF_CHUNK * 36;
            copy4_lds_untracked((const uint8_t*)msrc + (int64_t)c * PF_CHUNK * 4,
                                wave < 2 ? (void*)(s.xd + (wave & 1) * 64) : (void*)(s.xs + (wave & 1) * 64));
#pragma unroll
            for (int k = 0; k < NIT; k++) {
                const int c0 = wave * 64 + k * PF_THREADS;
                if (c0 < TWP) {
                    if (pval[k]) {
                        int64_t o = goff;
                        // span pieces stay in the row: column byte + chunk offset <= rb - 16
                        if constexpr (CBL != CB) o = goff + pcol[k] < rb - 16 ? goff : rb - 16 - pcol[k];
                        copy16_lds_untracked(psrc[k] + o, s.w + c0 * 16);
                    }
                } else if (c0 < TOT) {
                    if (pval[k]) copy16_lds_untracked(psrc[k] + xoff, s.x + (c0 - TWP) * 16);
                }
            }
        };
        // chunk c from stage cur, chunk c + 1 issued into nxt (the stage chunk
        // c - 1 was computed from: every wave has passed the barrier since)
        auto step = [&](int c, const PfStage& cur, const PfStage& nxt) {
            wait_vm<0>();
            lds_barrier();   // chunk c (weights, activations, metadata) landed: every wave's share
            if (c + 1 < nc) issue(c + 1, nxt);
            pf_mma_chunk<T, NTN, true>(cur.x, PF_XROW_AL, cur.xd, cur.xs, cur.w + wrow0 * CBLP + (c * CB & 15), CBLP,
                                       PF_CHUNK, grid, acc);
        };
        issue(0, s0);
        for (int c = 0; c < nc; c += 2) {
            step(c, s0, s1);
            if (c + 1 >= nc) break;
            step(c + 1, s1, s0);
        }
    }
    lds_barrier();   // every wave is done with the stages (callers reuse them)
}

// TWO: allow the two-stage path (callers whose rows are never 16-byte aligned
// pass false, so that the second stage's LDS is not allocated)
template <int T, int NTN, int NR, bool TWO = true>
__device__ __forceinline__ void pf_gemm(const PfStage& s0, const PfStage& s1, const uint8_t* w0, int n0,
                                        const uint8_t* w1, int64_t rb, int nbk, const uint8_t* xsrc,
                                        const int* xrows, int64_t xstride, const float* xmd, const int* xms,
                                        int wrow0, const uint32_t* grid, float (&acc)[NTN][4]) {
    // the two-stage path copies 16-byte pieces: rows and activations 16-byte aligned
    const bool al16 = (((uintptr_t)w0 | (uintptr_t)w1 | (uintptr_t)rb | (uintptr_t)xsrc | (uintptr_t)xstride) & 15) == 0;
    if constexpr (TWO)
        if (al16) {
            pf_gemm_k<T, NTN, NR, true>(s0, s1, w0, n0, w1, rb, nbk, xsrc, xrows, xstride, xmd, xms, wrow0, grid,
                                          acc);
            return;
        }
    // (the span copies only where the one-stage path is the path: on a
    // two-stage caller's rare fallback they would only add registers)
    pf_gemm_k<T, NTN, NR, false, !TWO>(s0, s1, w0, n0, w1, rb, nbk, xsrc, xrows, xstride, xmd, xms, wrow0, grid,
                                       acc);
}

template <int T>
constexpr int pf_wst(int nrows) { return nrows * pf_lds_row_al<T>() + 16; }
constexpr int PF_XST = PF_TILE * PF_XROW_AL;

// LDS arrays of the two pipeline stages (separate arrays) and their PfStage
#define PF_STAGE_ARRAYS(WS0, WS1)                                                                     \
    __shared__ __attribute__((aligned(16))) uint8_t wl0[WS0], wl1[WS1];                               \
    __shared__ __attribute__((aligned(16))) uint8_t xl0[PF_XST], xl1[PF_XST];                         \
    __shared__ __attribute__((aligned(16))) float xd0[PF_TILE * PF_CHUNK], xd1[PF_TILE * PF_CHUNK];   \
    __shared__ __attribute__((aligned(16))) int xs0[PF_TILE * PF_CHUNK], xs1[PF_TILE * PF_CHUNK];     \
    const PfStage s0{wl0, xl0, xd0, xs0}, s1{wl1, xl1, xd1, xs1}

// A Q8_0 or K-quant shared expert next to narrower expert rows (Q4_0 / IQ3_S
// experts) runs on one stage, so that the second stage is sized for the
// experts' chunk rows (two stages of 128 Q8_0 chunk rows leave one work-group
// per CU)
template <int TE, int TS>
constexpr bool pf_sh_one() { return (TS == T_Q8_0 || pf_kq<TS>() || TS == T_Q6_K) && TE != TS; }
template <int TE, int TS>
constexpr int pf_ws0(int nrows) { return pf_wst<TE>(nrows) > pf_wst<TS>(nrows) ? pf_wst<TE>(nrows) : pf_wst<TS>(nrows); }
template <int TE, int TS>
constexpr int pf_ws1(int nrows) { return pf_sh_one<TE, TS>() ? pf_wst<TE>(nrows) : pf_ws0<TE, TS>(nrows); }

// Rows per gate_up work-group: pf_gu_ntn 16-row tiles per wave, half the
// waves on gate rows and half on the same up rows.  IQ3_S experts: one tile
// per wave (64-row work-groups, 30-40 KB of LDS: four work-groups per CU;
// 512-token chunk 365 -> 354 us); the others two (measured alike or better).
template <int TE>
constexpr int pf_gu_ntn() { return TE == T_IQ3_S ? 1 : 2; }
template <int TE>
constexpr int pf_gu_rows() { return 32 * pf_gu_ntn<TE>(); }   // gate (and up) rows per work-group

// P4: grid (F/pf_gu_rows, max_tiles).  Waves 0, 1: gate and up rows f0 +
// [0, 16*NTN); waves 2, 3: the same for the next 16*NTN rows (NTN 16-row
// tiles per wave); then h = silu(gate) * up and Q8_1 of its 32-row blocks per
// pair.
template <int TE, int TS>
__global__ __launch_bounds__(PF_THREADS) void k_pf_gate_up(PfArgs a) {
    constexpr int NTN = pf_gu_ntn<TE>(), R = pf_gu_rows<TE>();
    constexpr int WS = pf_ws0<TE, TS>(2 * R);
    PF_STAGE_ARRAYS(WS, (pf_ws1<TE, TS>(2 * R)));
    __shared__ int prs[PF_TILE], xrows[PF_TILE];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    // gate / up results per (pair, row), in stage 0's weight buffer once the K loop is done
    static_assert(2 * PF_TILE * (R + 1) * sizeof(float) <= WS, "gate/up results fit a stage");
    float(*gu)[PF_TILE][R + 1] = reinterpret_cast<float(*)[PF_TILE][R + 1]>(wl0);
    const int ti = blockIdx.y;
    if (ti >= *a.ntiles) return;
    const int e = a.tiles[ti * 3], start = a.tiles[ti * 3 + 1], n = a.tiles[ti * 3 + 2];
    const int tid = threadIdx.x, TK = a.T * a.K;
    if (tid < PF_TILE) {
        const int p = a.spairs[start + min(tid, n - 1)];   // padding rows repeat the last pair
        prs[tid] = p;
        xrows[tid] = p < TK ? p / a.K : p - TK;
    }
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += PF_THREADS) grid[i] = c_iq3s_grid_pf[i];
    __syncthreads();
    const bool sh = e == a.E;
    const int f0 = blockIdx.x * R;
    const int wave = tid >> 6, mat = wave & 1, rh = wave >> 1;
    float acc[NTN][4];
    auto run = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        const int64_t rb = row_bytes(T, a.H);
        const uint8_t* g = sh ? a.sh_gate : a.gate + (int64_t)e * a.sg;
        const uint8_t* u = sh ? a.sh_up : a.up + (int64_t)e * a.su;
        pf_gemm<T, NTN, 2 * R, !(T == TS && pf_sh_one<TE, TS>())>(s0, s1, g + f0 * rb, R, u + f0 * rb, rb, a.H / QK,
                                                                 a.xq, xrows, a.xq_stride, a.xmd, a.xms,
                                                                 mat * R + rh * 16 * NTN, grid, acc);
    };
    if constexpr (TE == TS) run(std::integral_constant<int, TE>{});   // one instance of the K loop
    else if (!sh) run(std::integral_constant<int, TE>{});
    else run(std::integral_constant<int, TS>{});
    {
        const int lane = tid & 63, q = lane >> 4, c = lane & 15;
#pragma unroll
        for (int nn = 0; nn < NTN; nn++)
#pragma unroll
            for (int i = 0; i < 4; i++) gu[mat][4 * q + i][rh * 16 * NTN + 16 * nn + c] = acc[nn][i];
    }
    __syncthreads();
    // Q8_1(h) of the R/32 32-row blocks for each pair: one half-wave per (pair, block)
    constexpr int NBH = R / QK;
    for (int qq = tid >> 5; qq < NBH * n; qq += PF_THREADS / 32) {
        const int m = qq / NBH, blk = qq % NBH, i = tid & 31;
        const float xi = det_silu(gu[0][m][blk * 32 + i]) * gu[1][m][blk * 32 + i];
        const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
        const float d = amax / 127.0f;
        const int qv = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* o = a.hq + (int64_t)prs[m] * a.hq_stride + (f0 / QK + blk) * Q8_1_BYTES;
        o[4 + i] = (uint8_t)(int8_t)qv;
        // the block's metadata for the down launch (the quant sum is exact:
        // integers below 2^12 at every step of the float tree)
        const float sq = bfly32_sum((float)qv);
        if (i == 0) {
            const uint32_t dh = f2h(d);
            *(uint32_t*)o = dh | (f2h(sum) << 16);
            const int64_t mi = (int64_t)prs[m] * (a.hq_stride / Q8_1_BYTES) + f0 / QK + blk;
            a.hmd[mi] = h2f(dh);
            a.hms[mi] = -8 * (int)sq;
        }
    }
}

// 16-row tiles per wave of k_pf_down (64 * ntn rows per work-group): IQ3_S
// experts one (four work-groups per CU; 512-token chunk -5 us), the others
// two (alike)
template <int TE>
constexpr int pf_dn_ntn() { return TE == T_IQ3_S ? 1 : 2; }

// P5: grid (H/DR, max_tiles), DR = 128 (IQ3_S experts: 64, one 16-row tile
// per wave).  DR = 128: wave w: down rows r0 + 32w .. +31 (two
// 16-row tiles) for the tile's 16 pairs; K = F.
template <int TE, int TS>
__global__ __launch_bounds__(PF_THREADS) void k_pf_down(PfArgs a) {
    constexpr int NTN = pf_dn_ntn<TE>(), DR = 64 * NTN;
    PF_STAGE_ARRAYS((pf_ws0<TE, TS>(DR)), (pf_ws1<TE, TS>(DR)));
    __shared__ int prs[PF_TILE];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    const int ti = blockIdx.y;
    if (ti >= *a.ntiles) return;
    const int e = a.tiles[ti * 3], start = a.tiles[ti * 3 + 1], n = a.tiles[ti * 3 + 2];
    const int tid = threadIdx.x;
    if (tid < PF_TILE) prs[tid] = a.spairs[start + min(tid, n - 1)];
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += PF_THREADS) grid[i] = c_iq3s_grid_pf[i];
    __syncthreads();
    const bool sh = e == a.E;
    const int r0 = blockIdx.x * DR, wave = tid >> 6;
    float acc[NTN][4];
    auto run = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        const int64_t rb = row_bytes(T, a.F);
        const uint8_t* d = sh ? a.sh_down : a.down + (int64_t)e * a.sd;
        // IQ3_S / Q6_K down rows (F / 256 superblocks of 110 / 210 bytes) are
        // 16-byte aligned only when F is a multiple of 2048: one stage
        constexpr bool two = T != T_IQ3_S && T != T_Q6_K && !(T == TS && pf_sh_one<TE, TS>());
        pf_gemm<T, NTN, DR, two>(s0, s1, d + r0 * rb, DR, d, rb, a.F / QK, a.hq, prs, a.hq_stride, a.hmd, a.hms,
                                 wave * 16 * NTN, grid, acc);
    };
    if constexpr (TE == TS) run(std::integral_constant<int, TE>{});   // one instance of the K loop
    else if (!sh) run(std::integral_constant<int, TE>{});
    else run(std::integral_constant<int, TS>{});
    const int lane = tid & 63, q = lane >> 4, c = lane & 15;
#pragma unroll
    for (int nn = 0; nn < NTN; nn++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * q + i;
            if (m < n) a.dn[(int64_t)prs[m] * a.H + r0 + wave * 16 * NTN + 16 * nn + c] = acc[nn][i];
        }
}

// P6: grid (ceil(H/256), T): out = sum_k fmaf(w_k, dn_k, acc) (+ shared expert)
// one thread per 4 consecutive outputs of a token (H % 4 == 0, which every
// shape the prefill accepts has: H is a multiple of 256); each output's
// fmaf chain over k is the one of the decode layer's combine
__global__ __launch_bounds__(256) void k_pf_combine(PfArgs a) {
    const int t = blockIdx.y, h = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (h >= a.H) return;
    float4 v[MAX_K + 1];
#pragma unroll
    for (int k = 0; k < MAX_K; k++)
        if (k < a.K) v[k] = *(const float4*)(a.dn + (int64_t)(t * a.K + k) * a.H + h);
    if (a.has_shared) v[MAX_K] = *(const float4*)(a.dn + (int64_t)(a.T * a.K + t) * a.H + h);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < MAX_K; k++) {
        if (k < a.K) {
            const float w = a.wts[t * a.K + k];
            acc.x = __builtin_fmaf(w, v[k].x, acc.x);
            acc.y = __builtin_fmaf(w, v[k].y, acc.y);
            acc.z = __builtin_fmaf(w, v[k].z, acc.z);
            acc.w = __builtin_fmaf(w, v[k].w, acc.w);
        }
    }
    float4 o = acc;
    if (a.has_shared) {
        const float4 shv = v[MAX_K];
        if (a.sh_gate_w) {
            const float sg = 1.0f / (1.0f + det_exp(-a.glogit[t]));
            o = make_float4(__builtin_fmaf(shv.x, sg, acc.x), __builtin_fmaf(shv.y, sg, acc.y),
                            __builtin_fmaf(shv.z, sg, acc.z), __builtin_fmaf(shv.w, sg, acc.w));
        } else {
            o = make_float4(shv.x + acc.x, shv.y + acc.y, shv.z + acc.z, shv.w + acc.w);
        }
    }
    float* dst = a.out + (int64_t)t * a.H + h;
    if (((uintptr_t)a.out & 15) == 0) {
        *(float4*)dst = o;
    } else {   // a caller's output that is not 16-byte aligned
        dst[0] = o.x; dst[1] = o.y; dst[2] = o.z; dst[3] = o.w;
    }
}

void launch_quantize_q8_1(const float* x, void* out, int64_t ncols, int64_t ncols_padded, int64_t nrows,
                          hipStream_t s);

struct PfPlan {
    size_t logits, glogit, ids, wts, xq, spairs, tiles, ntiles, hq, dn, xmd, xms, hmd, hms, total;
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
    p.spairs = o; o += al256p(P * 4);
    p.tiles = o; o += al256p((size_t)p.max_tiles * 3 * 4);
    p.ntiles = o; o += al256p(4);
    p.hq = o; o += al256p(P * p.hq_stride);
    p.dn = o; o += al256p(P * H * 4);
    p.xmd = o; o += al256p((size_t)T * (p.xq_stride / Q8_1_BYTES) * 4);
    p.xms = o; o += al256p((size_t)T * (p.xq_stride / Q8_1_BYTES) * 4);
    p.hmd = o; o += al256p(P * (p.hq_stride / Q8_1_BYTES) * 4);
    p.hms = o; o += al256p(P * (p.hq_stride / Q8_1_BYTES) * 4);
    p.total = o;
    return p;
}

template <int TE, int TS>
static void launch_pf(const PfArgs& a, const PfPlan& p, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_router,
                       dim3(((a.E + (a.sh_gate_w ? 1 : 0) + PF_RE - 1) / PF_RE) * ((a.T + PF_RT - 1) / PF_RT)),
                       dim3(256), 0, s, a);
    launch_quantize_q8_1(a.x, a.xq, a.H, p.xq_stride / Q8_1_BYTES * QK, a.T, s);
    hipLaunchKernelGGL(k_pf_topk, dim3(a.T), dim3(64), 0, s, a);
    hipLaunchKernelGGL(k_pf_plan, dim3(1), dim3(1024), 0, s, a);
    hipLaunchKernelGGL((k_pf_gate_up<TE, TS>), dim3(a.F / pf_gu_rows<TE>(), p.max_tiles), dim3(PF_THREADS), 0, s, a);
    hipLaunchKernelGGL((k_pf_down<TE, TS>), dim3(a.H / (64 * pf_dn_ntn<TE>()), p.max_tiles), dim3(PF_THREADS), 0, s, a);
    hipLaunchKernelGGL(k_pf_combine, dim3((a.H / 4 + 255) / 256, a.T), dim3(256), 0, s, a);
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
    auto pf_type = [](int t) { return t == T_Q4_0 || t == T_Q8_0 || t == T_IQ3_S; };
    CHIMERE_REQUIRE(pf_type(L->expert_type) &&
                        (!has_sh || pf_type(L->shared_type) || L->shared_type == T_Q4_K || L->shared_type == T_Q5_K ||
                         L->shared_type == T_Q6_K),
                    CHIMERE_ERR_ARG,
                    "moe_prefill: Q4_0 / Q8_0 / IQ3_S experts, shared expert also Q4_K / Q5_K / Q6_K (expert %d, shared %d)",
                    L->expert_type, L->shared_type);
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
    a.xq = w + p.xq; a.spairs = (int*)(w + p.spairs);
    a.tiles = (int*)(w + p.tiles); a.ntiles = (int*)(w + p.ntiles);
    a.hq = w + p.hq; a.dn = (float*)(w + p.dn);
    a.xmd = (float*)(w + p.xmd); a.xms = (int*)(w + p.xms);
    a.hmd = (float*)(w + p.hmd); a.hms = (int*)(w + p.hms);
    a.xq_stride = p.xq_stride; a.hq_stride = p.hq_stride; a.max_tiles = p.max_tiles;
    const int te = L->expert_type, ts = has_sh ? L->shared_type : te;
    auto with_ts = [&](auto te_tag) {
        constexpr int TE = decltype(te_tag)::value;
        if (ts == T_Q4_0) launch_pf<TE, T_Q4_0>(a, p, stream);
        else if (ts == T_Q8_0) launch_pf<TE, T_Q8_0>(a, p, stream);
        else if (ts == T_Q4_K) launch_pf<TE, T_Q4_K>(a, p, stream);
        else if (ts == T_Q5_K) launch_pf<TE, T_Q5_K>(a, p, stream);
        else if (ts == T_Q6_K) launch_pf<TE, T_Q6_K>(a, p, stream);
        else launch_pf<TE, T_IQ3_S>(a, p, stream);
    };
    if (te == T_Q4_0) with_ts(std::integral_constant<int, T_Q4_0>{});
    else if (te == T_Q8_0) with_ts(std::integral_constant<int, T_Q8_0>{});
    else with_ts(std::integral_constant<int, T_IQ3_S>{});
    check_launch("moe_prefill");
}

}  // extern "C"
