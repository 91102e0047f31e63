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
//                     work-groups quantizing x to Q8_1 (8 blocks each).
//   K2 k_moe_expert   (distinct expert | shared) x (32-row block w of F).
//                     Each routed work-group recomputes softmax/top-k (one wave
//                     per token, registers only) and the distinct-expert plan
//                     from the logits, then streams 32 gate + 32 up rows and
//                     the block-w column slice of the down matrix together,
//                     once for all tokens routed to the expert, computes
//                     Q8_1(h) for its block and the exact down terms.
//   K3 k_moe_combine  replays the down dots' fp32 order from the terms, then
//                     the router-weighted sum in k order plus the shared
//                     expert.
// Every row dot uses the (L=16, G=1) order of tile_gemv.h.
#include <mutex>

#include "api_internal.h"
#include "common.h"
#include "tile_gemv.h"
#include "moe_common.h"

namespace chimere {

__constant__ uint32_t c_iq3s_grid_moe[512] = CHIMERE_IQ3S_GRID_INIT;

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
    uint2* terms;       // F > 512: [M*K + M][F/32][H]  down block terms (f32 scale bits, int32 sumi)
    float* lane_acc;    // F <= 512: [M*K + M][F/32][H]  lane j's finished accumulator (one block per lane)
    int64_t xq_stride;
    uint8_t* hq;        // M > 1: [M*K + M][hq_stride]  Q8_1(h) per pair
    float* dn;          // M > 1: [M*K + M][H]  down-projection output per pair (aliases terms)
    int64_t hq_stride;
};

// Published plan: [nu][uexp][untok][upair], then the items of the
// several-token gate/up launch: [ng] and ng entries {expert, ntok <= KG_NT,
// pair0, pair1} -- each unit's tokens in groups of KG_NT, units in order.
constexpr int KG_NT = 2;
constexpr int PLAN_UEXP = 1, PLAN_UNTOK = 1 + MAX_TOK * MAX_K, PLAN_UPAIR = 1 + 2 * MAX_TOK * MAX_K;
constexpr int PLAN_NG = PLAN_UPAIR + MAX_TOK * MAX_K * MAX_TOK, PLAN_GRP = PLAN_NG + 1;
constexpr int PLAN_INTS = PLAN_GRP + 4 * MAX_TOK * MAX_K;
static_assert(KG_NT == 2 && MAX_TOK <= 4 * KG_NT && MAX_TOK * MAX_K <= 128, "plan groups");

// Expert plan: distinct selected experts and, per expert, its (token, k) pairs.
struct Plan {
    int nu;
    int uexp[MAX_TOK * MAX_K];
    int untok[MAX_TOK * MAX_K];
    int upair[MAX_TOK * MAX_K][MAX_TOK];
    int utok[MAX_TOK * MAX_K][MAX_TOK];
};

// K1: grid (E + has_gate) * TS work-groups (router rows, then the
// shared-expert gate row; TS work-groups per row, each for NT of the tokens)
// + the x quantizers.
// HC: H as a compile-time constant (0: the run-time a.H)
template <int NT, int TS = 1, int HC = 0>
__global__ __launch_bounds__(256) void k_moe_route(MoeArgs a) {
    const int H = HC ? HC : a.H;
    __shared__ float red[NT * 256];
    const int ng = a.sh_gate_w ? 1 : 0;
    const int nrw = (a.E + ng) * TS;
    const int bid = blockIdx.x;
    const int row = bid < nrw ? bid / TS : a.E + ng + (bid - nrw);
    if (row >= a.E + ng) {
        // Q8_1(x): 8 blocks per work-group (one per half-wave), so that this
        // part of the grid finishes with the router rows
        const int nb = H / QK, qwg = (nb + 7) / 8;
        const int r = row - a.E - ng, t = r / qwg, b0 = (r - t * qwg) * 8;
        const float* xt = a.x + (int64_t)t * H + (int64_t)b0 * QK;
        uint8_t* dst = a.xq + t * a.xq_stride + b0 * Q8_1_BYTES;
        quantize_blocks(
            min(8, nb - b0), [&](int b, int i) { return xt[b * QK + i]; },
            [&](int b, int i, int q, float d, float sum) {
                uint8_t* blk = dst + b * Q8_1_BYTES;
                blk[4 + i] = (uint8_t)(int8_t)q;
                if (i == 0) *(uint32_t*)blk = f2h(d) | (f2h(sum) << 16);
            });
        return;
    }
    const int t0 = (bid - row * TS) * NT;
    if (t0 >= a.M) return;
    const int nt = min(NT, a.M - t0);
    float v[NT];
    const float* A = row < a.E ? a.router + (int64_t)row * H : a.sh_gate_w;
    f32_row_dot<NT>(A, a.x + (int64_t)t0 * H, H, nt, red, v);
    if (threadIdx.x == 0) {
        for (int t = 0; t < nt; t++) {
            if (row < a.E) a.logits[(t0 + t) * a.E + row] = a.bias ? v[t] + a.bias[row] : v[t];
            else a.glogit[t0 + t] = v[t];
        }
    }
}

constexpr int EX_RG = 64;                    // K2 row groups: 1024 threads
constexpr int EX_THREADS = EX_RG * SLOTS;
constexpr int EX_MAX_RPT = 4;                // down rows per thread: H <= 4096

// Loads, for the down rows of this thread, the weight block w (32 columns of
// F) of expert matrix `down` (row stride rbF).
template <int T>
__device__ __forceinline__ void load_down_blocks(RegBlk<T> (&rb)[EX_MAX_RPT], const uint8_t* down, int64_t rbF,
                                                 int w, int H) {
#pragma unroll
    for (int k = 0; k < EX_MAX_RPT; k++) {
        const int r = threadIdx.x + EX_THREADS * k;
        if (r < H) {
            const uint8_t* rowp = down + (int64_t)r * rbF;
            if constexpr (T == T_IQ3_S) rb[k].load(rowp + (w >> 3) * 110, w & 7);
            else rb[k].load(rowp + w * QTraits<T>::BYTES);
        }
    }
}

// Exact down-projection terms of block w for the thread's rows and every
// token of the unit.  F <= 512 (NB <= 16): lane w of the L=16 order owns only
// block w, so its finished accumulator fmaf(scale, sumi, 0) is stored
// (lane_acc[pair][w][r]); otherwise the term itself (terms[pair][w][r] =
// (f32(d_w) * f32(d_h), sumi)) for K3 to accumulate in order.
template <int T>
__device__ __forceinline__ void down_terms(const RegBlk<T> (&rb)[EX_MAX_RPT], const XLds* hx, const int* pairs,
                                           int ntok, const uint32_t* grid, const MoeArgs& a, int NB, int w) {
#pragma unroll
    for (int k = 0; k < EX_MAX_RPT; k++) {
        const int r = threadIdx.x + EX_THREADS * k;
        if (r < a.H) {
            WBlk wb;
            rb[k].decode(grid, wb);
            for (int t = 0; t < ntok; t++) {
                XBlk xb;
                xlds_to_blk(hx[t], xb);
                const int s = wdot<T>(wb, xb);
                const int64_t o = ((int64_t)pairs[t] * NB + w) * a.H + r;   // one contiguous run per block w
                if (NB <= SLOTS) a.lane_acc[o] = __builtin_fmaf(wb.dw * xb.d, (float)s, 0.0f);
                else a.terms[o] = make_uint2(__builtin_bit_cast(uint32_t, wb.dw * xb.d), (uint32_t)s);
            }
        }
    }
}

// Routing for all M tokens and the distinct-expert plan, by a 1024-thread
// work-group: waves 0..M-1 each run softmax/top-k for one token from the
// logits (registers only); then the plan is built in parallel: the first
// pair (lowest t*K+k) selecting an expert numbers it by its rank among first
// pairs; the order of pairs inside an expert does not affect any result.
// `first` is LDS scratch of E ints.  With `publish`, the routing weights
// (and ids_out / w_out) and the plan are written to global memory.
__device__ __forceinline__ void route_plan(const MoeArgs& a, int* first, Plan& pl, int* s_ids, float* s_w,
                                           bool publish, uint64_t (*tk)[128]) {
    const int tid = threadIdx.x;
    const int MK = a.M * a.K;

    const int wave = tid >> 6;
    if (wave < a.M)
        topk_wave_any(a.logits + wave * a.E, a.E, a.K, s_ids + wave * a.K, s_w + wave * a.K, tk[wave]);
    if (a.M == 1) {
        // one token: its K experts are distinct; unit k = the k-th selected
        __syncthreads();
        if (tid < MK) {
            pl.uexp[tid] = s_ids[tid];
            pl.untok[tid] = 1;
            pl.upair[tid][0] = tid;
            pl.utok[tid][0] = 0;
        }
        if (tid == 0) pl.nu = MK;
        __syncthreads();
    } else {
        // distinct-expert plan, built in parallel: the first pair (lowest
        // t*K+k) selecting an expert numbers it by its rank among first pairs;
        // the order of pairs inside an expert does not affect any result.
        __shared__ int s_fcnt[2], s_cnt[MAX_TOK * MAX_K];
        for (int e = tid; e < a.E; e += (int)blockDim.x) first[e] = 0x7fffffff;
        if (tid < MAX_TOK * MAX_K) s_cnt[tid] = 0;
        __syncthreads();
        if (tid < MK) atomicMin(&first[s_ids[tid]], tid);
        __syncthreads();
        int fp = 0;
        bool isfirst = false;
        if (tid < 128) {
            fp = tid < MK ? first[s_ids[tid]] : -1;
            isfirst = tid < MK && fp == tid;
            const uint64_t m = __ballot(isfirst);
            if ((tid & 63) == 0) s_fcnt[tid >> 6] = __popcll(m);
            const int lrank = __popcll(m & ((1ull << (tid & 63)) - 1));
            __syncthreads();
            const int rank = lrank + ((tid >> 6) ? s_fcnt[0] : 0);
            if (isfirst) { pl.uexp[rank] = s_ids[tid]; s_cnt[tid] = rank; }   // s_cnt: first pair -> unit
            if (tid == 0) pl.nu = s_fcnt[0] + (MK > 64 ? s_fcnt[1] : 0);
        } else {
            __syncthreads();
        }
        __syncthreads();
        int uu = 0;
        if (tid < MK) uu = s_cnt[fp];
        __syncthreads();
        if (tid < MAX_TOK * MAX_K) s_cnt[tid] = 0;
        __syncthreads();
        if (tid < MK) {
            const int n = atomicAdd(&s_cnt[uu], 1);
            pl.upair[uu][n] = tid;
            pl.utok[uu][n] = tid / a.K;
        }
        __syncthreads();
        if (tid < pl.nu) pl.untok[tid] = s_cnt[tid];
        __syncthreads();
    }
    if (publish) {
        const int nu = pl.nu;
        for (int i = tid; i < MK; i += (int)blockDim.x) {
            a.wts[i] = s_w[i];
            if (a.ids_out) { a.ids_out[i] = s_ids[i]; a.w_out[i] = s_w[i]; }
        }
        int* P = a.plan;
        if (tid == 0) P[0] = nu;
        for (int i = tid; i < nu; i += (int)blockDim.x) {
            P[PLAN_UEXP + i] = pl.uexp[i];
            P[PLAN_UNTOK + i] = pl.untok[i];
            for (int n = 0; n < pl.untok[i]; n++) P[PLAN_UPAIR + i * MAX_TOK + n] = pl.upair[i][n];
        }
        // gate/up items: unit i's ceil(untok / KG_NT) groups start at the
        // number of groups of units < i (per-wave ballot counts; nu <= 128)
        __shared__ int s_gtot[2];
        int g = 0, pre = 0;
        if (tid < 128) {
            g = tid < nu ? (pl.untok[tid] + KG_NT - 1) / KG_NT : 0;
            const uint64_t lt = (1ull << (tid & 63)) - 1;
            int tot = 0;
#pragma unroll
            for (int k = 1; k <= MAX_TOK / KG_NT; k++) {
                const uint64_t m = __ballot(g >= k);
                pre += __popcll(m & lt);
                tot += __popcll(m);
            }
            if ((tid & 63) == 0) s_gtot[tid >> 6] = tot;
        }
        __syncthreads();
        if (tid < 128) {
            if (tid >= 64) pre += s_gtot[0];
            if (tid == 0) P[PLAN_NG] = s_gtot[0] + s_gtot[1];
            for (int k = 0; k < g; k++) {
                int* q = P + PLAN_GRP + 4 * (pre + k);
                const int t0 = KG_NT * k, n = min(KG_NT, pl.untok[tid] - t0);
                q[0] = pl.uexp[tid];
                q[1] = n;
                q[2] = pl.upair[tid][t0];
                q[3] = n > 1 ? pl.upair[tid][t0 + 1] : 0;
            }
        }
    }

}

// One work item of K2 (see below): gate/up rows [32w, 32w+32) of one expert
// (weights of type T at gate / up / down), h block w, and its down terms.
template <int T, int NT, int CB>
__device__ __forceinline__ void expert_item(const MoeArgs& a, uint8_t* tile, XLds (*xs)[MAX_CHUNK_BLOCKS],
                                            const uint32_t* grid, float (*hg)[QK], float (*hu)[QK], XLds* hx,
                                            const int* toks, const int* pairs, int ntok, int w, const uint8_t* gate,
                                            const uint8_t* up, const uint8_t* down) {
    const int tid = threadIdx.x;
    const int NB = a.F / QK;
    const int r0 = w * QK;
    RegBlk<T> db[EX_MAX_RPT];
    float acc[1][NT];
    const int64_t rb = row_bytes(T, a.H);
    tile_gemv<T, NT, EX_RG, 1>(tile, &xs[0][0], grid, gate + r0 * rb, QK, up + r0 * rb, QK, rb, a.H, a.xq, a.xq_stride, toks,
                               ntok, acc);
    // the down column slice is requested only now, behind the gate/up rows
    // (its pieces are prefetched into L2 by the idle work-groups of this XCD)
    load_down_blocks<T>(db, down, row_bytes(T, a.F), w, a.H);
    const int g = tid >> 4, j = tid & 15;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (t < ntok) {
            const float v = slot_reduce16(acc[0][t]);
            if (j == 0) {
                if (g < QK) hg[t][g] = v;
                else hu[t][g - QK] = v;
            }
        }
    }
    __syncthreads();
    // one half-wave per token: Q8_1 of the 32-row block of h (ggml
    // semantics), kept decoded in LDS for the down terms
    if ((tid >> 5) < ntok) {
        const int t = tid >> 5, i = tid & 31;
        const float xi = det_silu(hg[t][i]) * hu[t][i];
        const float amax = bfly32_max(__builtin_fabsf(xi));
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        const int byte = (q & 0xFF) << (8 * (i & 3));
        int word = byte | xlane<1>(byte);
        word = word | xlane<2>(word);
        int sq = q + xlane<16>(q);
        sq = sq + xlane<8>(sq);
        sq = sq + xlane<4>(sq);
        sq = sq + xlane<2>(sq);
        sq = sq + xlane<1>(sq);
        if ((i & 3) == 0) hx[t].q[i >> 2] = word;
        if (i == 0) { hx[t].d = h2f(f2h(d)); hx[t].sumq = sq; }
    }
    __syncthreads();
    down_terms<T>(db, hx, pairs, ntok, grid, a, NB, w);
}

// K2: work items (unit, w): unit = a distinct selected expert (or the shared
// expert), w = a 32-row block of its F dimension.  1024 threads; the grid is
// at most one work-group per CU and each work-group loops over items
// V = blockIdx.x, blockIdx.x + gridDim.x, ...
//  1. Routing, once per work-group: waves 0..M-1 each run softmax/top-k for
//     one token from the logits (registers only), then the distinct-expert
//     plan.  No work-group waits on another: each recomputes it; work-group 0
//     publishes weights and plan for K3.
//  Per item:
//  2. Issues, together: the 32 gate + 32 up rows of block w (HBM -> LDS,
//     asynchronous) and the block-w column slice of the down matrix (one
//     weight block per down row, into registers).
//  3. gate/up dots (group g < 32: gate row g, 32 + g: up row g), h =
//     silu(gate)*up, Q8_1(h) for the 32-row block (ggml semantics).
//  4. Exact down terms of block w for every down row (the L=16 order needs
//     only these per-block (scale, sumi) pairs; K3 replays the order).
// Item V goes to XCD V & 7 (the grid is a multiple of 8 and work-group ids
// are dealt round-robin to the 8 XCDs); consecutive units of an XCD's items
// are 8 apart, so one expert's row blocks share that XCD's L2.
template <int TE, int TS, int NT>
__global__ __launch_bounds__(EX_THREADS) void k_moe_expert(MoeArgs a) {
    constexpr int CBE = ChunkGeom<TE>::BYTES, CBS = ChunkGeom<TS>::BYTES;
    constexpr int CB = CBE > CBS ? CBE : CBS;
    constexpr int TILE_BYTES = EX_RG * CB + 16 > MAX_E * 4 ? EX_RG * CB + 16 : MAX_E * 4;
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE_BYTES];
    __shared__ XLds xs[NT][MAX_CHUNK_BLOCKS];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ float hg[MAX_TOK][QK], hu[MAX_TOK][QK];
    __shared__ XLds hx[MAX_TOK];
    __shared__ int toks[MAX_TOK], pairs[MAX_TOK];
    __shared__ int s_ids[MAX_TOK * MAX_K];
    __shared__ float s_w[MAX_TOK * MAX_K];
    __shared__ Plan pl;
    __shared__ uint64_t s_tk[NT][128];

    const int NB = a.F / QK;
    const int MK = a.M * a.K;
    const int tid = threadIdx.x;
    route_plan(a, (int*)tile, pl, s_ids, s_w, blockIdx.x == 0, s_tk);
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += EX_THREADS) grid[i] = c_iq3s_grid_moe[i];
    // Items of XCD x (work-groups b with b % 8 == x): the row blocks of the
    // routed units u = x, x+8, ... then the shared unit's blocks w = x, x+8, ...
    // Work-groups without an item prefetch the down matrices those items read
    // (their column slices are scattered 18..34-byte pieces: from L2 they cost
    // only the per-request issue time, from HBM a full memory latency each).
    const int x = blockIdx.x & 7, lb = blockIdx.x >> 3, G8 = gridDim.x >> 3;
    const int nr = pl.nu > x ? (pl.nu - 1 - x) / 8 + 1 : 0;
    const int ns = a.has_shared ? (NB > x ? (NB - 1 - x) / 8 + 1 : 0) : 0;
    const int nx = nr * NB + ns;
    if (lb >= nx) {
        // helper: first the up rows of this XCD's items (requested by the items
        // right behind their gate rows), then the down matrices; each helper
        // takes an equal contiguous share of both, one 2-byte load per 64 bytes
        // (weights are 2-byte aligned)
        const int nh = G8 - nx, hb = lb - nx;
        uint32_t sink = 0;
        const int64_t LE = QK * row_bytes(TE, a.H), LS = QK * row_bytes(TS, a.H);
        const int64_t ua = (int64_t)nr * NB * LE + ns * LS;
        for (int64_t o = ua * hb / nh + 64 * (int64_t)tid, e1 = ua * (hb + 1) / nh; o < e1; o += 64 * EX_THREADS) {
            const int64_t rl = (int64_t)nr * NB * LE;
            const uint8_t* p;
            if (o < rl) {
                const int i = (int)(o / LE);
                p = a.up + (int64_t)pl.uexp[x + 8 * (i / NB)] * a.su + (int64_t)(i % NB) * LE + (o - (int64_t)i * LE);
            } else {
                const int j = (int)((o - rl) / LS);
                p = a.sh_up + (int64_t)(x + 8 * j) * LS + (o - rl - (int64_t)j * LS);
            }
            sink += *(const uint16_t*)((uintptr_t)p & ~(uintptr_t)1);
        }
        const int64_t mb = (int64_t)a.H * row_bytes(TE, a.F), sb = (int64_t)a.H * row_bytes(TS, a.F);
        const int64_t total = nr * mb + (ns ? sb : 0);
        for (int64_t o = total * hb / nh + 64 * (int64_t)tid, e1 = total * (hb + 1) / nh; o < e1; o += 64 * EX_THREADS) {
            const int m = (int)(o / mb);
            const uint8_t* base = m < nr ? a.down + (int64_t)pl.uexp[x + 8 * m] * a.sd : a.sh_down;
            const int64_t off = m < nr ? o - (int64_t)m * mb : o - (int64_t)nr * mb;
            sink += *(const uint16_t*)(base + (off & ~(int64_t)1));
        }
        if (a.H < 0) a.plan[0] = (int)sink;   // never taken: keeps the loads
        return;
    }
    for (int i = lb; i < nx; i += G8) {
        const bool shared = i >= nr * NB;
        const int u = shared ? MK : x + 8 * (i / NB);
        const int w = shared ? x + 8 * (i - nr * NB) : i % NB;
        const int ntok = shared ? a.M : pl.untok[u];
        __syncthreads();   // the previous item's readers of toks / pairs / hx are done
        if (tid < ntok) {
            toks[tid] = shared ? tid : pl.utok[u][tid];
            pairs[tid] = shared ? MK + tid : pl.upair[u][tid];
        }
        if (shared)
            expert_item<TS, NT, CB>(a, tile, xs, grid, hg, hu, hx, toks, pairs, ntok, w, a.sh_gate, a.sh_up, a.sh_down);
        else
            expert_item<TE, NT, CB>(a, tile, xs, grid, hg, hu, hx, toks, pairs, ntok, w, a.gate + pl.uexp[u] * a.sg,
                                    a.up + pl.uexp[u] * a.su, a.down + pl.uexp[u] * a.sd);
    }
}

// ------------------------------------------ one token, common shapes: K2'
// k_moe_expert1 does K2's work for one token when every work-group holds at
// most one item and the weight rows are 16-byte aligned (Q4_0 / Q8_0 experts,
// Q4_0 / Q8_0 / Q4_K / Q5_K shared expert, hidden <= 2048, ffn <= 512,
// top_k <= 8): the same items, fp32 order and outputs, laid out for latency.
//  * The shared expert's items do not wait for routing; the routed items'
//    Q8_1(x) blocks are decoded by waves 1.. while wave 0 runs softmax/top-k.
//  * Gate/up rows arrive in K chunks alternating between two LDS buffers, so
//    the dots of one chunk overlap the copy of the next.  Wave w copies rows
//    w, w+16, w+32, w+48 of a chunk (one asynchronous copy instruction per
//    row), so every thread issues E1_ROWS copies per chunk and "chunk c has
//    landed" is vmcnt <= E1_ROWS (copies of chunk c+1 outstanding).
//  * The down column slice is requested behind the first two chunks, so its
//    latency overlaps the gate/up dots.
constexpr int E1_ROWS = 2 * QK / (EX_THREADS / 64);   // rows copied per wave and chunk: 4
template <int T>
constexpr int e1_cblk() { return T == T_Q8_0 ? 16 : 32; }   // blocks per chunk
template <int T>
constexpr int e1_cbytes() { return chunk_bytes<T>(e1_cblk<T>()); }
// LDS row stride of a chunk: IQ3_S chunks (4 superblocks, 440 B) are copied as
// the 16-byte aligned span holding them, up to 15 bytes more on each side
// (<= 470 B), in 576-byte rows: 144 dwords, so rows g and g+4 land 64 banks
// apart and the 16 lanes of one row read banks apart from the neighbouring
// rows' (measured: 1.2 % off the IQ3_S one-token layer against 464 B rows)
template <int T>
constexpr int e1_stride() { return T == T_IQ3_S ? 576 : e1_cbytes<T>(); }
static_assert((e1_cbytes<T_IQ3_S>() + 15 + 15) / 16 * 16 <= e1_stride<T_IQ3_S>(), "IQ3_S span fits its row");
constexpr int E1_MAX_H = 2048;

// Copies chunk c (blocks [c*CBLK, c*CBLK + cb)) of the 2*QK gate/up rows into
// buf (row stride e1_stride).  One copy instruction per (wave, row).  Rows
// start 16-byte aligned; a chunk that does not (IQ3_S) is copied as the
// 16-byte aligned span holding it and starts `pre` bytes into its LDS row
// (the same for every row): the return value.
template <int T>
__device__ __forceinline__ int e1_issue(uint8_t* buf, const uint8_t* gate, const uint8_t* up, int64_t rb, int c,
                                        int nbH) {
    constexpr int CBLK = e1_cblk<T>();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cb = min(CBLK, nbH - c * CBLK);
    const int64_t goff = chunk_bytes<T>(c * CBLK);
    const int pre = (int)(goff & 15);
    const int span = pre + chunk_bytes<T>(cb);   // bytes from the aligned start
#pragma unroll
    for (int k = 0; k < E1_ROWS; k++) {
        const int r = wave + (EX_THREADS / 64) * k;
        const uint8_t* src = (r < QK ? gate + (int64_t)r * rb : up + (int64_t)(r - QK) * rb) + goff - pre;
        if (lane * 16 < span)
            __builtin_amdgcn_global_load_lds((const glb_void_t*)(src + lane * 16),
                                             (lds_void_t*)(buf + r * e1_stride<T>()), 16, 0, CPOL_STREAM);
    }
    return pre;
}

// k_moe_expert1's items decode IQ3_S with the sign-folded codebook: 36 of
// the ~70 VALU instructions of a block's decode (the per-word sign masks) go
// for ~8 more of index arithmetic; the 32 KiB fill overlaps the logits /
// top-k phase, and the kernel's one work-group per CU has the LDS.  One-token
// IQ3_S layer 16.86 -> 16.76 us (Q5_K shared), 16.75 -> 16.61 us (Q8_0); in
// the several-token and prefill kernels, whose LDS it crowds and whose fill
// it cannot hide, the same table was slower.
constexpr bool E1_SG = true;
// Dots of chunk c for this thread's row (row group g) and lane j: blocks
// j, j+16, ... of the chunk, in ascending order (the L=16 order).
template <int T>
__device__ __forceinline__ float e1_dots(const uint8_t* buf, int pre, const XLds* xs, const uint32_t* grid, int c,
                                         int nbH, float acc) {
    constexpr int CBLK = e1_cblk<T>();
    const int g = threadIdx.x >> 4, j = threadIdx.x & 15;
    const int cb = min(CBLK, nbH - c * CBLK);
    const uint8_t* row = buf + g * e1_stride<T>() + pre;
#pragma unroll
    for (int b = j; b < CBLK; b += SLOTS) {
        if (b < cb) {
            WBlk wb;
            block_decode<T, E1_SG>(row, b, grid, wb);
            XBlk xb;
            xlds_to_blk(xs[c * CBLK + b], xb);
            acc = wacc<T>(wb, xb, acc);
        }
    }
    return acc;
}

// The item: gate/up rows [32w, 32w+32) of one expert, h block w, and its down
// terms (lane_acc[pair][w][r], F <= 512).
template <int T, int HC>
__device__ __forceinline__ void e1_item(const MoeArgs& a, uint8_t* bufA, uint8_t* bufB, const XLds* xs,
                                        const uint32_t* grid, float (*hg)[QK], float (*hu)[QK], int pair, int w,
                                        const uint8_t* gate, const uint8_t* up) {
    constexpr int CBLK = e1_cblk<T>();
    const int tid = threadIdx.x;
    const int nbH = (HC ? HC : a.H) / QK;
    const int nc = (nbH + CBLK - 1) / CBLK;
    const int64_t rb = row_bytes(T, nbH * QK);
    gate += (int64_t)w * QK * rb;
    up += (int64_t)w * QK * rb;
    int preA = e1_issue<T>(bufA, gate, up, rb, 0, nbH), preB = 0;
    if (nc > 1) preB = e1_issue<T>(bufB, gate, up, rb, 1, nbH);
    // in issue order: chunk 0, chunk 1, then chunk c+2 while chunk c+1 is
    // computed; chunk c has landed when at most the copies of the chunk after
    // it are outstanding
    float acc = 0.0f;
    for (int c = 0; c < nc; c += 2) {
        if (c + 1 < nc) wait_vm<E1_ROWS>();
        else wait_vm<0>();
        lds_barrier();
        acc = e1_dots<T>(bufA, preA, xs, grid, c, nbH, acc);
        if (c + 1 >= nc) break;
        lds_barrier();   // every wave is done with buffer A
        if (c + 2 < nc) {
            preA = e1_issue<T>(bufA, gate, up, rb, c + 2, nbH);
            wait_vm<E1_ROWS>();
        } else {
            wait_vm<0>();
        }
        lds_barrier();
        acc = e1_dots<T>(bufB, preB, xs, grid, c + 1, nbH, acc);
        if (c + 2 >= nc) break;
        lds_barrier();   // every wave is done with buffer B
        if (c + 3 < nc) preB = e1_issue<T>(bufB, gate, up, rb, c + 3, nbH);
    }
    const int g = tid >> 4, j = tid & 15;
    const float v = slot_reduce16(acc);
    if (j == 0) {
        if (g < QK) hg[0][g] = v;
        else hu[0][g - QK] = v;
    }
    __syncthreads();
    // one half-wave: Q8_1 of the 32-row block w of h (ggml semantics), to
    // the pair's row of hq for the down projection
    if (tid < 32) {
        const int i = tid;
        const float xi = det_silu(hg[0][i]) * hu[0][i];
        const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* o = a.hq + (int64_t)pair * a.hq_stride + w * Q8_1_BYTES;
        o[4 + i] = (uint8_t)(int8_t)q;
        if (i == 0) *(uint32_t*)o = f2h(d) | (f2h(sum) << 16);
    }
}

// Helper work-groups of k_moe_expert1 (those without an item) prefetch the
// down rows that the down/combine launch reads on their XCD: rows
// [x H/8, (x+1) H/8) of every pair's down matrix (mb / sb: bytes of an
// expert's / the shared down matrix), one 2-byte load per 64 bytes, each
// helper an equal contiguous share.  (Prefetching the items' own up rows as
// well was measured slower: it only adds traffic next to the items' requests.)
// helpers' wait before their down-row loads, in ticks of the 100 MHz
// constant clock (s_memrealtime): 2 us
constexpr uint64_t E1_HELPER_DELAY = 200;

struct E1Prefetch {
    const uint8_t *down, *sh_down;
    int64_t sd, mb, sb;
    int K, has_shared;
    int* sink_dst;
};

__device__ __forceinline__ void e1_prefetch(const E1Prefetch& p, const int* uexp, int x, int hb, int nh) {
    uint32_t sink = 0;
    const int64_t sE = p.mb / 8, sS = p.sb / 8;
    const int64_t total = (int64_t)p.K * sE + (p.has_shared ? sS : 0);
    for (int64_t o = total * hb / nh + 64 * (int64_t)threadIdx.x, e1 = total * (hb + 1) / nh; o < e1;
         o += 64 * EX_THREADS) {
        const int m = (int)(o / sE);
        const uint8_t* base = m < p.K ? p.down + (int64_t)uexp[m] * p.sd + x * sE : p.sh_down + x * sS;
        const int64_t off = m < p.K ? o - (int64_t)m * sE : o - (int64_t)p.K * sE;
        sink += *(const uint16_t*)(base + (off & ~(int64_t)1));
    }
    if (p.K < 0) *p.sink_dst = (int)sink;   // never taken: keeps the loads
}

// HC / FC: H and F as compile-time constants (0: the run-time a.H / a.F);
// the shapes of the reference model run an instance with both fixed.
template <int TE, int TS, int HC = 0, int FC = 0>
__global__ __launch_bounds__(EX_THREADS) void k_moe_expert1(MoeArgs a) {
    constexpr int CB = e1_stride<TE>() > e1_stride<TS>() ? e1_stride<TE>() : e1_stride<TS>();
    // + 16: lds_u32 of a row's last block reads up to 4 bytes past the row
    __shared__ __attribute__((aligned(16))) uint8_t bufA[2 * QK * CB + 16];
    __shared__ __attribute__((aligned(16))) uint8_t bufB[2 * QK * CB + 16];
    __shared__ __attribute__((aligned(16))) uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? (E1_SG ? 8192 : 512) : 1];
    __shared__ XLds xs[E1_MAX_H / QK];
    __shared__ float hg[1][QK], hu[1][QK];
    __shared__ int s_ids[MAX_K];
    __shared__ float s_w[MAX_K];
    __shared__ uint64_t s_tk[128];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int Hs = HC ? HC : a.H, Fs = FC ? FC : a.F;
    const int NB = Fs / QK, nbH = Hs / QK;
    const int x = blockIdx.x & 7, lb = blockIdx.x >> 3, G8 = gridDim.x >> 3;
    // items of XCD x (work-group ids are dealt round-robin to the 8 XCDs): the
    // row blocks of the routed unit x (the x-th selected expert), then the
    // shared expert's blocks x, x+8, ...; the rest are helpers
    const int nr = a.K > x ? 1 : 0;
    const int ns = a.has_shared ? (NB > x ? (NB - 1 - x) / 8 + 1 : 0) : 0;
    const int nx = nr * NB + ns;
    const bool routed = lb < nr * NB, shared = !routed && lb < nx;
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S) {   // visible after the first barrier below
        if constexpr (E1_SG) {
            if (routed || shared) iq3s_sgrid_fill(grid, tid, EX_THREADS);
        } else {
            for (int i = tid; i < 512; i += EX_THREADS) grid[i] = c_iq3s_grid_moe[i];
        }
    }
    if (!shared) {
        // wave 0: softmax / top-k; the other waves decode Q8_1(x) meanwhile
        if (wave == 0) {
            topk_wave_any(a.logits, a.E, a.K, s_ids, s_w, s_tk);
            if (blockIdx.x == 0 && tid < a.K) {
                a.wts[tid] = s_w[tid];
                a.plan[PLAN_UEXP + tid] = s_ids[tid];
                if (a.ids_out) { a.ids_out[tid] = s_ids[tid]; a.w_out[tid] = s_w[tid]; }
            }
        } else if (routed) {
            for (int i = tid - 64; i < nbH; i += EX_THREADS - 64) {
                XBlk xb;
                load_xblk(a.xq + (int64_t)i * Q8_1_BYTES, xb);
                xs[i].d = xb.d; xs[i].sumq = xb.sumq;
#pragma unroll
                for (int k = 0; k < 8; k++) xs[i].q[k] = xb.q[k];
            }
        }
        __syncthreads();
        if (!routed) {
            const int nh = G8 - nx, hb = lb - nx;
            E1Prefetch p;
            p.down = a.down; p.sh_down = a.sh_down; p.sd = a.sd;
            p.mb = (int64_t)Hs * row_bytes(TE, Fs); p.sb = (int64_t)Hs * row_bytes(TS, Fs);
            p.K = a.K; p.has_shared = a.has_shared;
            p.sink_dst = a.plan;
            {   // start the down-row loads once the items' gate/up copies are
                // under way: issued together they share HBM with the copies
                // on the critical path (layer 15.06 -> 14.55 us; 1.5 - 2.5 us
                // measured alike)
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                while (__builtin_amdgcn_s_memrealtime() - t0 < E1_HELPER_DELAY) __builtin_amdgcn_s_sleep(2);
            }
            e1_prefetch(p, s_ids, x, hb, nh);
            return;
        }
        const int e = s_ids[x];
        e1_item<TE, HC>(a, bufA, bufB, xs, grid, hg, hu, x, lb, a.gate + e * a.sg, a.up + e * a.su);
    } else {
        for (int i = tid; i < nbH; i += EX_THREADS) {
            XBlk xb;
            load_xblk(a.xq + (int64_t)i * Q8_1_BYTES, xb);
            xs[i].d = xb.d; xs[i].sumq = xb.sumq;
#pragma unroll
            for (int k = 0; k < 8; k++) xs[i].q[k] = xb.q[k];
        }
        e1_item<TS, HC>(a, bufA, bufB, xs, grid, hg, hu, a.K, x + 8 * (lb - nr * NB), a.sh_gate, a.sh_up);
    }
}

// K3: grid (ceil(H/16)), 256 threads: 16 down rows per work-group, 16 lanes
// per row.  Lane j replays the L=16 order for every (token, k) pair from the
// exact block terms (acc = fmaf(scale_b, sumi_b, acc) over b = j, j+16, ...,
// then the halving tree), then the router-weighted sum in k order plus the
// shared expert.
constexpr int CMB_CHUNK = 16;   // pairs whose terms are loaded together

__global__ __launch_bounds__(GEMV_THREADS) void k_moe_combine(MoeArgs a) {
    __shared__ float s_w[MAX_TOK * MAX_K];
    __shared__ float s_g[MAX_TOK];
    __shared__ float dn[TILE_ROWS][MAX_TOK * MAX_K + MAX_TOK];
    const int tid = threadIdx.x;
    const int rr = tid >> 4, j = tid & 15;
    // neighbouring 16-row tiles on one XCD (work-group b runs on XCD b % 8):
    // they share the 128-byte lines of the block-major terms
    const int tile_i = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
    const int r = tile_i * TILE_ROWS + rr;
    const int NB = a.F / QK;
    const int MK = a.M * a.K;
    for (int i = tid; i < MK; i += GEMV_THREADS) s_w[i] = a.wts[i];
    if (tid < a.M) s_g[tid] = a.sh_gate_w ? a.glogit[tid] : 0.0f;
    const int np = MK + (a.has_shared ? a.M : 0);
    if (r < a.H) {
        for (int p0 = 0; p0 < np; p0 += CMB_CHUNK) {
            float accs[CMB_CHUNK];
            if (NB <= SLOTS) {
                // one block per lane: the stored value is the lane's accumulator
#pragma unroll
                for (int c = 0; c < CMB_CHUNK; c++)
                    accs[c] = (p0 + c < np && j < NB) ? a.lane_acc[((int64_t)(p0 + c) * NB + j) * a.H + r] : 0.0f;
            } else {
                // issue every term load of the chunk before using any
                uint2 tv[CMB_CHUNK][EX_MAX_RPT];
#pragma unroll
                for (int c = 0; c < CMB_CHUNK; c++)
#pragma unroll
                    for (int q = 0; q < EX_MAX_RPT; q++) {
                        const int b = j + SLOTS * q;
                        tv[c][q] = (p0 + c < np && b < NB) ? a.terms[((int64_t)(p0 + c) * NB + b) * a.H + r]
                                                           : make_uint2(0, 0);
                    }
#pragma unroll
                for (int c = 0; c < CMB_CHUNK; c++) {
                    float acc = 0.0f;
#pragma unroll
                    for (int q = 0; q < EX_MAX_RPT; q++)
                        if (j + SLOTS * q < NB)
                            acc = __builtin_fmaf(__builtin_bit_cast(float, tv[c][q].x), (float)(int)tv[c][q].y, acc);
                    accs[c] = acc;
                }
            }
#pragma unroll
            for (int c = 0; c < CMB_CHUNK; c++) {
                if (p0 + c < np) {
                    const float v = slot_reduce16(accs[c]);
                    if (j == 0) dn[rr][p0 + c] = v;
                }
            }
        }
    }
    __syncthreads();
    // combine: one thread per (row, token)
    if (tid < TILE_ROWS * a.M) {
        const int row = tid % TILE_ROWS, t = tid / TILE_ROWS;
        const int rg = tile_i * TILE_ROWS + row;
        if (rg < a.H) {
            float acc = 0.0f;
            for (int k = 0; k < a.K; k++) acc = __builtin_fmaf(s_w[t * a.K + k], dn[row][t * a.K + k], acc);
            float o = acc;
            if (a.has_shared) {
                const float sh = dn[row][MK + t];
                if (a.sh_gate_w) o = __builtin_fmaf(sh, 1.0f / (1.0f + det_exp(-s_g[t])), acc);
                else o = sh + acc;
            }
            a.out[(int64_t)t * a.H + rg] = o;
        }
    }
}

// K3' (with k_moe_expert1): down projection and combine for one token.
// Grid H/4 work-groups of np*64 threads (np = K routed pairs in rank order,
// then the shared expert): wave p takes pair p for the work-group's 4 down
// rows, 16 lanes per row; lane j takes block j of the row (F <= 512: one
// block per lane) against the pair's Q8_1(h) block j, so the row's value is
// the L=16 halving tree of fmaf(f32(d_w) * f32(d_h), sumi, 0) -- the value K3
// rebuilds from K2's lane terms.  Then the router-weighted sum in k order plus
// the shared expert.  Work-group b runs on XCD b % 8 and takes the b/8-th
// tile of XCD b % 8's contiguous row range.
constexpr int DC1_ROWS = 4;

template <int T>
__device__ __forceinline__ float dc1_row(const uint8_t* row, int j, const uint8_t* hblk, const uint32_t* grid,
                                         bool act) {
    RegBlk<T> rbk;
    uint32_t hw[9];
    if (act) {
        if constexpr (T == T_IQ3_S) rbk.load(row + (j >> 3) * 110, j & 7);
        else rbk.load(row + j * QTraits<T>::BYTES);
        const uint32_t* h = (const uint32_t*)hblk;
#pragma unroll
        for (int k = 0; k < 9; k++) hw[k] = h[k];
    }
    float v = 0.0f;
    if (act) {
        WBlk w;
        rbk.decode(grid, w);
        XBlk xb;
        xb.d = h2f(hw[0] & 0xFFFFu);
        int sq = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) { xb.q[k] = (int)hw[1 + k]; sq = dot4(xb.q[k], 0x01010101, sq); }
        xb.sumq = sq;
        v = wacc<T>(w, xb, 0.0f);
    }
    return slot_reduce16(v);
}

template <int T>
constexpr bool is_kquant() { return T == T_Q4_K || T == T_Q5_K || T == T_Q6_K; }

// K-quant shared expert (256-element superblocks whose blocks are spread over
// the superblock): the wave stages its 4 rows in LDS with 2-byte loads, then
// each lane decodes its block from there.
template <int T>
__device__ __forceinline__ float dc1_row_lds(uint8_t* rows, const uint8_t* d0, int64_t rbF, int rr, int j,
                                             const uint8_t* hblk, bool act) {
    const int lane = threadIdx.x & 63;
    XBlk xb;
    if (act) load_xblk(hblk, xb);
    // the DC1_ROWS rows are contiguous: 16-byte pieces where the weights are
    // 16-byte aligned (Q4_K / Q5_K rows at F = 512: 288 / 352 bytes), else
    // 2-byte pieces (the boundary only promises 2-byte aligned weights)
    const int nb = (int)(DC1_ROWS * rbF);
    if ((((uintptr_t)d0 | (uintptr_t)nb) & 15) == 0) {
        for (int i = lane; i < nb / 16; i += 64) ((uint4*)rows)[i] = ((const uint4*)d0)[i];
    } else {
        for (int i = lane; i < nb / 2; i += 64) ((uint16_t*)rows)[i] = ((const uint16_t*)d0)[i];
    }
    float v = 0.0f;
    if (act) {
        WBlk w;
        block_decode<T>(rows + rr * rbF, j, nullptr, w);
        v = wacc<T>(w, xb, 0.0f);
    }
    return slot_reduce16(v);
}

// k_moe_dc1 runs only where expert1_fits holds (top_k <= E1_MAX_K)
constexpr int E1_MAX_K = 8;
static_assert((E1_MAX_K + 2) * 64 <= 1024, "dc1 work-group size");

// FC: F as a compile-time constant (0: the run-time a.F)
template <int TE, int TS, int FC = 0>
__global__ __launch_bounds__((E1_MAX_K + 2) * 64) void k_moe_dc1(MoeArgs a) {
    __shared__ float dn[DC1_ROWS][E1_MAX_K + 1];
    __shared__ float s_wk[E1_MAX_K + 1];   // routing weights, then the shared-expert gate logit
    __shared__ __attribute__((aligned(16))) uint8_t srows[is_kquant<TS>() ? DC1_ROWS * 2 * 256 : 1];   // F <= 512
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    const int tid = threadIdx.x, j = tid & 15, rr = (tid >> 4) & (DC1_ROWS - 1), p = tid >> 6;
    const int tile_i = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
    const int r = tile_i * DC1_ROWS + rr;
    const int F = FC ? FC : a.F;
    const int NB = F / QK, K = a.K;
    const bool act = j < NB && r < a.H;
    const uint8_t* hb = a.hq + (int64_t)p * a.hq_stride + j * Q8_1_BYTES;
    float v = 0.0f;
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S) {
        for (int i = tid; i < 512; i += blockDim.x) grid[i] = c_iq3s_grid_moe[i];
        __syncthreads();
    }
    if (p == K + a.has_shared) {
        // the last wave only reads the routing weights and the gate logit
        // (results of the previous launch) into LDS, so that no pair's
        // down-row loads queue behind them and the combine finds them there
        const int lane = tid & 63;
        if (lane < K) s_wk[lane] = a.wts[lane];
        else if (lane == K && a.has_shared && a.sh_gate_w) s_wk[K] = a.glogit[0];
    } else if (p < K) {
        const int e = a.plan[PLAN_UEXP + p];
        v = dc1_row<TE>(a.down + (int64_t)e * a.sd + (int64_t)r * row_bytes(TE, F), j, hb, grid, act);
    } else if constexpr (is_kquant<TS>()) {
        const int64_t rbF = row_bytes(TS, F);
        v = dc1_row_lds<TS>(srows, a.sh_down + (int64_t)tile_i * DC1_ROWS * rbF, rbF, rr, j, hb, act);
    } else {
        v = dc1_row<TS>(a.sh_down + (int64_t)r * row_bytes(TS, F), j, hb, grid, act);
    }
    if (j == 0 && p < K + a.has_shared) dn[rr][p] = v;
    __syncthreads();
    if (tid < DC1_ROWS) {
        const int rg = tile_i * DC1_ROWS + tid;
        if (rg < a.H) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = __builtin_fmaf(s_wk[k], dn[tid][k], acc);
            float o = acc;
            if (a.has_shared) {
                const float sh = dn[tid][K];
                if (a.sh_gate_w) o = __builtin_fmaf(sh, 1.0f / (1.0f + det_exp(-s_wk[K])), acc);
                else o = sh + acc;
            }
            a.out[rg] = o;
        }
    }
}

// ------------------------------------------------ several tokens (M > 1)
// With M > 1 the work per selected expert grows with its token count, so the
// layer runs as five launches that each keep many work-groups in flight:
// K1 router (as above), KP routing + plan (one work-group), KG gate/up + SiLU
// + Q8_1(h) per (expert, 32-row block of F), KD down GEMV per (expert, 64-row
// tile of H) with every h block of the expert's tokens (each output row
// reduced in the L=16 order in place), KC router-weighted combine.

// one wave per token (M <= 8): 512 threads
constexpr int PLAN_THREADS = MAX_TOK * 64;
static_assert(PLAN_THREADS >= MAX_TOK * MAX_K, "one thread per pair");
__global__ __launch_bounds__(PLAN_THREADS) void k_moe_plan(MoeArgs a) {
    __shared__ int first[MAX_E];
    __shared__ Plan pl;
    __shared__ int s_ids[MAX_TOK * MAX_K];
    __shared__ float s_w[MAX_TOK * MAX_K];
    __shared__ uint64_t s_tk[MAX_TOK][128];
    route_plan(a, first, pl, s_ids, s_w, true, s_tk);
}

// unit u of the published plan (u == M*K: the shared expert); false if none
__device__ __forceinline__ bool load_unit(const MoeArgs& a, int u, int* pairs, int* toks, int& ntok, int64_t& e) {
    const int MK = a.M * a.K;
    if (u == MK) {
        if (!a.has_shared) return false;
        ntok = a.M;
        e = -1;
        if (threadIdx.x < a.M) { pairs[threadIdx.x] = MK + threadIdx.x; toks[threadIdx.x] = threadIdx.x; }
        return true;
    }
    if (u >= a.plan[0]) return false;
    ntok = a.plan[PLAN_UNTOK + u];
    e = a.plan[PLAN_UEXP + u];
    if (threadIdx.x < ntok) {
        const int p = a.plan[PLAN_UPAIR + u * MAX_TOK + threadIdx.x];
        pairs[threadIdx.x] = p;
        toks[threadIdx.x] = p / a.K;
    }
    return true;
}

constexpr int KG_RG = 16;     // KG / KD: 256 threads, 64 rows per tile (4 per row group)
// blocks per chunk: the tile and 8 tokens' blocks fit three work-groups per CU
constexpr int KG_CHUNK = 32;
template <int T>
constexpr int kg_chunk() { return T == T_Q8_0 ? 16 : KG_CHUNK; }
// KG: K chunks of 16 blocks, double-buffered where two 64-row buffers of
// kg_buf bytes fit (Q4_0, Q4_K: 288-byte rows; IQ3_S: 240-byte slots for the
// 16-byte aligned spans of its 220-byte chunks); Q8_0 / Q5_K / Q6_K rows are
// single-buffered.  Each item carries at most KG_NT tokens, so the tile, two
// tokens' activation chunks, the codebook and h fit in 40 KB: four
// work-groups per CU, and a decode batch's items (M = 8: up to 64 routed
// groups + 4 shared ones, 16 blocks each) start in one round.
constexpr int KG_BLK = 16;
constexpr int KG_BUF = 64 * 16 * 18 + 16;
template <int T>
constexpr int kg_buf() { return T == T_IQ3_S ? 64 * 16 * 15 + 16 : KG_BUF; }
template <int T>
constexpr bool kg_db() { return 64 * chunk_bytes<T>(KG_BLK) + 16 <= kg_buf<T>(); }
template <int T>
constexpr int kg_tile_bytes() { return kg_db<T>() ? 2 * kg_buf<T>() : 64 * chunk_bytes<T>(KG_BLK) + 16; }

template <int T>
__device__ __forceinline__ void kg_tile(uint8_t* tile, XLds* xs, uint8_t* xraw, const uint32_t* grid, const uint8_t* g,
                                        const uint8_t* u, int64_t rb, const MoeArgs& a, const int* toks, int ntok,
                                        float (&acc)[4][KG_NT]) {
    if (ntok == 1) {   // most experts of a decode batch serve one token: no token loop
        float a1[4][1];
        if constexpr (kg_db<T>())
            tile_gemv_db<T, 1, KG_RG, 4, KG_BLK, CPOL_STREAM>(tile, kg_buf<T>(), xraw, grid, g, QK, u, QK, rb, a.H,
                                                              a.xq, a.xq_stride, toks, 1, a1);
        else
            tile_gemv<T, 1, KG_RG, 4, KG_BLK, CPOL_STREAM>(tile, xs, grid, g, QK, u, QK, rb, a.H, a.xq, a.xq_stride, toks, 1, a1);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r][0] = a1[r][0];
        return;
    }
    if constexpr (kg_db<T>())
        tile_gemv_db<T, KG_NT, KG_RG, 4, KG_BLK, CPOL_STREAM>(tile, kg_buf<T>(), xraw, grid, g, QK, u, QK, rb, a.H, a.xq,
                                                              a.xq_stride, toks, ntok, acc);
    else
        tile_gemv<T, KG_NT, KG_RG, 4, KG_BLK, CPOL_STREAM>(tile, xs, grid, g, QK, u, QK, rb, a.H, a.xq, a.xq_stride, toks,
                                                           ntok, acc);
}

// KG: grid NB * (SG + M*K), SG = ceil(M / KG_NT) shared groups (0 without a
// shared expert).  Work-group V takes group q = V / NB, block w = V % NB:
// groups q < SG are the shared expert's tokens [KG_NT q, KG_NT q + KG_NT),
// the rest the plan's gate/up items (groups past the plan's count exit).
// Consecutive work-groups run on consecutive XCDs, so the items spread evenly
// over the 8 XCDs, and the groups of one unit (same weight rows, 16 work-groups
// apart) on one XCD, close in time.
template <int TE, int TS>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_gateup(MoeArgs a) {
    constexpr int TILE = kg_tile_bytes<TE>() > kg_tile_bytes<TS>() ? kg_tile_bytes<TE>() : kg_tile_bytes<TS>();
    __shared__ __attribute__((aligned(16))) uint8_t tile[TILE];
    // raw Q8_1 blocks (double-buffered path) or decoded blocks (single-buffered path)
    static_assert(KG_NT * KG_BLK * sizeof(XLds) <= 2 * KG_NT * KG_BLK * Q8_1_BYTES, "xbuf");
    __shared__ __attribute__((aligned(16))) uint8_t xraw[2 * KG_NT * KG_BLK * Q8_1_BYTES];
    XLds* xs = (XLds*)xraw;
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ float hg[KG_NT][QK], hu[KG_NT][QK];
    __shared__ int toks[KG_NT], pairs[KG_NT];
    const int NB = a.F / QK, MK = a.M * a.K;
    const int SG = a.has_shared ? (a.M + KG_NT - 1) / KG_NT : 0;
    const int q = blockIdx.x / NB, w = blockIdx.x - q * NB;
    const int tid = threadIdx.x;
    int ntok;
    int64_t e;
    if (q < SG) {
        e = -1;
        ntok = min(KG_NT, a.M - KG_NT * q);
        if (tid < ntok) { toks[tid] = KG_NT * q + tid; pairs[tid] = MK + KG_NT * q + tid; }
    } else {
        const int qq = q - SG;
        if (qq >= a.plan[PLAN_NG]) return;
        const int* G = a.plan + PLAN_GRP + 4 * qq;
        e = G[0];
        ntok = G[1];
        if (tid < ntok) {
            const int p = G[2 + tid];
            pairs[tid] = p;
            toks[tid] = p / a.K;
        }
    }
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_moe[i];
    // toks / pairs (written by the first ntok threads) are read by every wave
    // in the tile's first copy, which precedes the tile's first barrier
    __syncthreads();
    float acc[4][KG_NT];
    const int r0 = w * QK;
    if (e < 0) {
        const int64_t rb = row_bytes(TS, a.H);
        kg_tile<TS>(tile, xs, xraw, grid, a.sh_gate + r0 * rb, a.sh_up + r0 * rb, rb, a, toks, ntok, acc);
    } else {
        const int64_t rb = row_bytes(TE, a.H);
        kg_tile<TE>(tile, xs, xraw, grid, a.gate + e * a.sg + r0 * rb, a.up + e * a.su + r0 * rb, rb, a, toks, ntok,
                    acc);
    }
    // group g holds tile rows g, g+16 (gate rows) and g+32, g+48 (up rows)
    const int g = tid >> 4, j = tid & 15;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int t = 0; t < KG_NT; t++) {
            if (t < ntok) {
                const float v = slot_reduce16(acc[r][t]);
                if (j == 0) {
                    const int row = g + KG_RG * r;
                    if (row < QK) hg[t][row] = v;
                    else hu[t][row - QK] = v;
                }
            }
        }
    __syncthreads();
    // one half-wave per token: Q8_1 of the 32-row block w of h (ggml semantics)
    for (int t = tid >> 5; t < ntok; t += GEMV_THREADS / 32) {
        const int i = tid & 31;
        const float xi = det_silu(hg[t][i]) * hu[t][i];
        const float amax = bfly32_max(__builtin_fabsf(xi)), sum = bfly32_sum(xi);
        const float d = amax / 127.0f;
        const int q8 = amax == 0.0f ? 0 : (int)__builtin_roundf(xi / d);
        uint8_t* o = a.hq + (int64_t)pairs[t] * a.hq_stride + w * Q8_1_BYTES;
        o[4 + i] = (uint8_t)(int8_t)q8;
        if (i == 0) *(uint32_t*)o = f2h(d) | (f2h(sum) << 16);
    }
}

template <int T>
__device__ __forceinline__ void kd_tile(uint8_t* tile, XLds* xs, const uint32_t* grid,
                                        const uint8_t* rows, int nr, int64_t rb, const MoeArgs& a, const int* pairs,
                                        int ntok, float (&acc)[4][MAX_TOK]) {
    if (ntok == 1) {
        float a1[4][1];
        tile_gemv<T, 1, KG_RG, 4, kg_chunk<T>(), CPOL_STREAM>(tile, xs, grid, rows, nr, nullptr, 0, rb, a.F, a.hq, a.hq_stride,
                                                 pairs, 1, a1);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r][0] = a1[r][0];
        return;
    }
    tile_gemv<T, MAX_TOK, KG_RG, 4, kg_chunk<T>(), CPOL_STREAM>(tile, xs, grid, rows, nr, nullptr, 0, rb, a.F, a.hq,
                                                   a.hq_stride, pairs, ntok, acc);
}

// KD: grid (H/64, M*K+1): down rows [64*blockIdx.x, +64) of unit blockIdx.y - 1 (y = 0: shared expert).
template <int TE, int TS>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_down(MoeArgs a) {
    constexpr int CBE = chunk_bytes<TE>(kg_chunk<TE>()), CBS = chunk_bytes<TS>(kg_chunk<TS>());
    constexpr int CB = CBE > CBS ? CBE : CBS;
    __shared__ __attribute__((aligned(16))) uint8_t tile[4 * KG_RG * CB + 16];
    __shared__ XLds xs[MAX_TOK * KG_CHUNK];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ int toks[MAX_TOK], pairs[MAX_TOK];
    int ntok;
    int64_t e;
    // unit blockIdx.y - 1; y = 0: the shared expert (heaviest, dispatched first)
    if (!load_unit(a, blockIdx.y == 0 ? a.M * a.K : (int)blockIdx.y - 1, pairs, toks, ntok, e)) return;
    const int tid = threadIdx.x;
    if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
        for (int i = tid; i < 512; i += GEMV_THREADS) grid[i] = c_iq3s_grid_moe[i];
    const int r0 = blockIdx.x * 4 * KG_RG, nr = min(4 * KG_RG, a.H - r0);
    float acc[4][MAX_TOK];
    // the h rows are indexed by pair
    if (e < 0) {
        const int64_t rb = row_bytes(TS, a.F);
        kd_tile<TS>(tile, xs, grid, a.sh_down + r0 * rb, nr, rb, a, pairs, ntok, acc);
    } else {
        const int64_t rb = row_bytes(TE, a.F);
        kd_tile<TE>(tile, xs, grid, a.down + e * a.sd + r0 * rb, nr, rb, a, pairs, ntok, acc);
    }
    const int g = tid >> 4, j = tid & 15;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int t = 0; t < MAX_TOK; t++) {
            if (t < ntok) {
                const float v = slot_reduce16(acc[r][t]);
                const int row = g + KG_RG * r;
                if (j == 0 && row < nr) a.dn[(int64_t)pairs[t] * a.H + r0 + row] = v;
            }
        }
}

// KC: grid (ceil(H/256), M): out = sum_k fmaf(w_k, dn_k, acc) in k order (+ shared expert)
__global__ __launch_bounds__(256) void k_moe_combine_dn(MoeArgs a) {
    const int t = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
    if (h >= a.H) return;
    const int MK = a.M * a.K;
    float acc = 0.0f;
    for (int k = 0; k < a.K; k++)
        acc = __builtin_fmaf(a.wts[t * a.K + k], a.dn[(int64_t)(t * a.K + k) * a.H + h], acc);
    float o = acc;
    if (a.has_shared) {
        const float sh = a.dn[(int64_t)(MK + t) * a.H + h];
        if (a.sh_gate_w) o = __builtin_fmaf(sh, 1.0f / (1.0f + det_exp(-a.glogit[t])), acc);
        else o = sh + acc;
    }
    a.out[(int64_t)t * a.H + h] = o;
}

// KDC: down projection and combine in one launch (M > 1, F == KDC_F), used
// where every unit's rows fit: grid H / DR work-groups of 1024 threads, each
// owning DR output rows.  All selected units' DR down rows (one contiguous
// run of DR * row_bytes per unit) and every pair's Q8_1(h) row are copied to
// LDS, so the whole layer's down bytes are in flight at once (one work-group
// per CU).  The work is in tasks -- a weight row against its tokens -- for
// the 64 groups of 16 lanes: lane j decodes weight block j of the row and,
// for each token, forms fmaf(d_w * d_h, sumi, 0) against h block j, summed
// over the 16 lanes by the halving tree (the L=16 order with one block per
// lane, F = 512).  The shared expert's (row, token) tasks run first, while
// the routed runs are in flight; then each wave works on the units whose runs
// it copied, unit by unit as they land (its own copies, so its in-order copy
// counter tells it; no barrier), its 4 groups taking rows g, g+4, ...
// Last, each (token, row) output is the router-weighted sum in k order plus
// the shared expert, as in k_moe_combine_dn.
constexpr int KDC_F = 512, KDC_THREADS = 1024, KDC_MAX_UNITS = 64;
constexpr int KDC_HQ = KDC_F / QK * Q8_1_BYTES;   // bytes of one pair's Q8_1(h) row (the hq stride)
template <int T>
constexpr int kdc_rb() { return KDC_F / QTraits<T>::ELEMS * QTraits<T>::BYTES; }
// rows per work-group: the routed runs of KDC_MAX_UNITS units within ~110 KB
template <int T>
constexpr int kdc_rows() { return KDC_MAX_UNITS * 8 * kdc_rb<T>() <= 112640 ? 8 : (KDC_MAX_UNITS * 4 * kdc_rb<T>() <= 112640 ? 4 : 2); }

// both runs (routed and shared) whole 16-byte pieces
template <int TE, int TS>
constexpr bool kdc_types() {
    return (TE == T_IQ3_S || TE == T_Q4_0 || TE == T_Q8_0) && kdc_rows<TE>() * kdc_rb<TE>() % 16 == 0 &&
           kdc_rows<TE>() * kdc_rb<TS>() % 16 == 0;
}

template <int TE, int TS>
__global__ __launch_bounds__(KDC_THREADS) void k_moe_down_comb(MoeArgs a) {
    constexpr int DR = kdc_rows<TE>();
    constexpr int RUNE = DR * kdc_rb<TE>(), RUNS = DR * kdc_rb<TS>();
    static_assert(RUNE % 16 == 0 && RUNS % 16 == 0 && KDC_HQ % 16 == 0, "16-byte runs");
    constexpr int PE = RUNE / 16, PS = RUNS / 16, PH = KDC_HQ / 16;
    // weights: the shared run at 0, routed run u at RUNS + u * RUNE; + 16:
    // lds_u32 of a row's last block reads up to 4 bytes past the row
    __shared__ __attribute__((aligned(16))) uint8_t wl[RUNS + KDC_MAX_UNITS * RUNE + 16];
    __shared__ __attribute__((aligned(16))) uint8_t hl[(KDC_MAX_UNITS + MAX_TOK) * KDC_HQ];
    __shared__ float dn[(KDC_MAX_UNITS + MAX_TOK) * DR];
    __shared__ uint32_t grid[(TE == T_IQ3_S || TS == T_IQ3_S) ? 512 : 1];
    __shared__ int s_uexp[KDC_MAX_UNITS];
    __shared__ uint8_t s_untok[KDC_MAX_UNITS], s_upair[KDC_MAX_UNITS][MAX_TOK];   // pair ids < 128
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * DR;
    const int MK = a.M * a.K, NP = MK + (a.has_shared ? a.M : 0);
    // Copies in three regions, each starting on a 64-piece round so that a
    // wave's 64 pieces never straddle two (the LDS base of a copy instruction
    // is wave-uniform; lanes past a region's end skip).  Wave 0 reads the plan
    // and the IQ3_S codebook into LDS while waves 1.. issue the pairs' h rows
    // (contiguous in hq) and the shared run; after an LDS-only barrier every
    // wave issues the routed runs.  The copies are untracked (their wait is
    // the explicit vmcnt(0) below): a tracked copy would make each later wait
    // of the same wave -- and __syncthreads() -- wait for all of them, since
    // the counter is in order.
    const int nh = NP * PH, nsp = a.has_shared ? PS : 0;
    const int th = (nh + 63) & ~63, ts = th + ((nsp + 63) & ~63);
    constexpr int NW = KDC_THREADS / 64;
    if (wave == 0) {
        // the plan's first KDC_MAX_UNITS units, read without waiting for its count
        s_uexp[lane] = a.plan[PLAN_UEXP + lane];
        s_untok[lane] = (uint8_t)a.plan[PLAN_UNTOK + lane];
#pragma unroll
        for (int i = lane; i < KDC_MAX_UNITS * MAX_TOK; i += 64)
            s_upair[i / MAX_TOK][i % MAX_TOK] = (uint8_t)a.plan[PLAN_UPAIR + i];
        if constexpr (TE == T_IQ3_S || TS == T_IQ3_S)
#pragma unroll
            for (int i = lane; i < 512; i += 64) grid[i] = c_iq3s_grid_moe[i];
    } else {
        for (int c0 = (wave - 1) * 64; c0 < ts; c0 += (NW - 1) * 64) {
            const int i = c0 + lane;
            if (c0 < th) {
                if (i < nh) copy16_lds_untracked(a.hq + (int64_t)i * 16, hl + c0 * 16);
            } else if (i - th < nsp) {
                copy16_lds_untracked(a.sh_down + (int64_t)r0 * kdc_rb<TS>() + (i - th) * 16, wl + (c0 - th) * 16);
            }
        }
    }
    lds_barrier();
    const int nu = a.plan[0];
    // routed runs: wave w copies units w, w + NW, ... (a unit's source and
    // destination bases are wave-uniform; lane l copies pieces l, l + 64, ...):
    // NPW copy instructions per unit, issued after the wave's h / shared ones
    constexpr int NPW = (PE + 63) / 64;
    static_assert(NPW * ((KDC_MAX_UNITS + NW - 1) / NW) <= 15, "copy counter");
    for (int u = wave; u < nu; u += NW) {
        const uint8_t* src = a.down + (int64_t)s_uexp[u] * a.sd + (int64_t)r0 * kdc_rb<TE>();
        uint8_t* dst = wl + RUNS + u * RUNE;
#pragma unroll
        for (int c0 = 0; c0 < PE; c0 += 64)
            if (c0 + lane < PE) copy16_lds_untracked(src + (c0 + lane) * 16, dst + c0 * 16);
    }
    const int nown = nu > wave ? (nu - wave + NW - 1) / NW : 0;   // units this wave copied
    wait_vm_n(NPW * nown);   // this wave's h / shared copies have landed
    lds_barrier();           // ... and every wave's
    const int g = tid >> 4, j = tid & 15;
    // one (weight row, tokens) task: pairs pr[0..ntok) against row r
    auto task = [&](auto tag, const uint8_t* row, int r, int ntok, auto pair_of) {
        constexpr int T = decltype(tag)::value;
        WBlk wb;
        block_decode<T>(row, j, grid, wb);
#pragma unroll
        for (int t = 0; t < MAX_TOK; t++) {
            if (t < ntok) {
                const int p = pair_of(t);
                XBlk xb;
                load_xblk(hl + p * KDC_HQ + j * Q8_1_BYTES, xb);
                const float v = slot_reduce16(wacc<T>(wb, xb, 0.0f));
                if (j == 0) dn[p * DR + r] = v;
            }
        }
    };
    // the shared expert's (row, token) tasks over all groups
    const int nsh = a.has_shared ? DR * a.M : 0;
    for (int k = g; k < nsh; k += KDC_THREADS / 16) {
        const int r = k / a.M, t = k - r * a.M;
        task(std::integral_constant<int, TS>{}, wl + r * kdc_rb<TS>(), r, 1, [&](int) { return MK + t; });
    }
    // this wave's units, each once its runs have landed
    for (int i = 0; i < nown; i++) {
        const int u = wave + NW * i;
        wait_vm_n(NPW * (nown - 1 - i));
        // the group's rows (DR / 4 of them, or one) unrolled: independent
        // decodes the compiler can interleave
#pragma unroll
        for (int ri = 0; ri < (DR + 3) / 4; ri++) {
            const int r = (g & 3) + 4 * ri;
            if (DR % 4 != 0 && r >= DR) break;   // DR = 2: groups 2 and 3 have no row
            task(std::integral_constant<int, TE>{}, wl + RUNS + u * RUNE + r * kdc_rb<TE>(), r, (int)s_untok[u],
                 [&](int t) { return (int)s_upair[u][t]; });
        }
    }
    __syncthreads();
    if (tid < a.M * DR) {
        const int t = tid / DR, r = tid - t * DR, h = r0 + r;
        if (h < a.H) {
            float acc = 0.0f;
            for (int k = 0; k < a.K; k++) acc = __builtin_fmaf(a.wts[t * a.K + k], dn[(t * a.K + k) * DR + r], acc);
            float o = acc;
            if (a.has_shared) {
                const float sh = dn[(MK + t) * DR + r];
                if (a.sh_gate_w) o = __builtin_fmaf(sh, 1.0f / (1.0f + det_exp(-a.glogit[t])), acc);
                else o = sh + acc;
            }
            a.out[(int64_t)t * a.H + h] = o;
        }
    }
}

// k_moe_down_comb's conditions: F == 512, at most KDC_MAX_UNITS units, H a
// multiple of the row count, 16-byte aligned runs
static bool kdc_fits(const MoeArgs& a, int te, int ts) {
    if (a.F != KDC_F || a.M * a.K > KDC_MAX_UNITS || a.M > MAX_TOK) return false;
    const int rbe = (int)row_bytes(te, KDC_F), rbs = (int)row_bytes(ts, KDC_F);
    const int dr = te == T_IQ3_S ? 8 : (te == T_Q4_0 ? 4 : 2);   // kdc_rows<TE>()
    const uintptr_t al = (uintptr_t)a.down | (uintptr_t)a.sd | (uintptr_t)(dr * rbe) |
                         (a.has_shared ? ((uintptr_t)a.sh_down | (uintptr_t)(dr * rbs)) : 0);
    return a.H % dr == 0 && (al & 15) == 0 && a.hq_stride == KDC_HQ && ((uintptr_t)a.hq & 15) == 0;
}

// ------------------------------------------------------- workspace plan

struct WsPlan {
    size_t logits, glogit, wts, plan, xq, terms, hq, total;
    int64_t xq_stride, hq_stride;
};

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

static WsPlan plan_ws(int H, int F, int E, int K, int M) {
    WsPlan p{};
    size_t o = 0;
    const int P = M * K + M;
    p.xq_stride = pad_to(H, ROW_PAD) / QK * Q8_1_BYTES;
    p.logits = o; o += al256((size_t)M * E * 4);
    p.glogit = o; o += al256((size_t)M * 4);
    p.wts = o; o += al256((size_t)M * K * 4);
    p.plan = o; o += al256((size_t)PLAN_INTS * 4);
    p.xq = o; o += al256((size_t)M * p.xq_stride);
    p.terms = o; o += al256((size_t)P * H * (F / QK) * (F / QK <= SLOTS ? 4 : 8));
    p.hq_stride = pad_to(F, ROW_PAD) / QK * Q8_1_BYTES;
    p.hq = o; o += al256((size_t)P * p.hq_stride);
    p.total = o;
    return p;
}

// K1 grid: router rows (+ the shared-expert gate row) and 8 Q8_1 blocks of x
// per work-group
constexpr int ROUTE_TS = 4;   // several-token router: work-groups per row
static int route_grid(const MoeArgs& a, int ts = 1) {
    return (a.E + (a.sh_gate_w ? 1 : 0)) * ts + a.M * ((a.H / QK + 7) / 8);
}


// K2 grid: all items, capped at one work-group per CU (a multiple of 8)
static int expert_grid(int items) {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
        cus[dev] = n / 8 * 8;
    }
    return items < cus[dev] ? items : cus[dev];
}

// k_moe_expert1's conditions: one item per work-group, 16-byte aligned rows
static bool expert1_fits(const MoeArgs& a, int te, int ts) {
    const int NB = a.F / QK;
    const int ns = a.has_shared ? (NB + 7) / 8 : 0;
    const uintptr_t al = (uintptr_t)a.gate | (uintptr_t)a.up | (uintptr_t)a.down | (uintptr_t)a.sg |
                         (uintptr_t)a.su | (uintptr_t)a.sd | (uintptr_t)a.sh_gate | (uintptr_t)a.sh_up |
                         (uintptr_t)a.sh_down | (uintptr_t)a.xq | (uintptr_t)row_bytes(te, a.H) |
                         (uintptr_t)(a.has_shared ? row_bytes(ts, a.H) : 0);
    return a.M == 1 && a.K <= E1_MAX_K && a.H <= E1_MAX_H && NB <= SLOTS && (al & 15) == 0 &&
           NB + ns <= expert_grid(256) / 8;
}

// stage < 0: all three kernels; 0, 1, 2: only K1, K2 or K3
template <int TE, int TS, int NT>
static void launch_layer_nt(const MoeArgs& a, int stage, hipStream_t s) {
    if (stage < 0 || stage == 0) {
        if (a.H == 2048) hipLaunchKernelGGL((k_moe_route<NT, 1, 2048>), dim3(route_grid(a)), dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_moe_route<NT>), dim3(route_grid(a)), dim3(256), 0, s, a);
    }
    if constexpr (NT == 1 && (TE == T_Q4_0 || TE == T_Q8_0 || TE == T_IQ3_S) &&
                  (TS == T_Q4_0 || TS == T_Q8_0 || TS == T_IQ3_S || TS == T_Q4_K || TS == T_Q5_K)) {
        if (expert1_fits(a, TE, TS)) {
            if (stage < 0 || stage == 1) {
                if (a.H == 2048 && a.F == 512)
                    hipLaunchKernelGGL((k_moe_expert1<TE, TS, 2048, 512>), dim3(expert_grid(256)), dim3(EX_THREADS), 0,
                                       s, a);
                else
                    hipLaunchKernelGGL((k_moe_expert1<TE, TS>), dim3(expert_grid(256)), dim3(EX_THREADS), 0, s, a);
            }
            if (stage < 0 || stage == 2) {
                if (a.F == 512)
                    hipLaunchKernelGGL((k_moe_dc1<TE, TS, 512>), dim3(a.H / DC1_ROWS),
                                       dim3((a.K + a.has_shared + 1) * 64), 0, s, a);
                else
                    hipLaunchKernelGGL((k_moe_dc1<TE, TS>), dim3(a.H / DC1_ROWS), dim3((a.K + a.has_shared + 1) * 64),
                                       0, s, a);
            }
            return;
        }
    }
    if constexpr (!is_kquant<TS>()) {
        if (stage < 0 || stage == 1)
            hipLaunchKernelGGL((k_moe_expert<TE, TS, NT>), dim3(expert_grid(256)), dim3(EX_THREADS), 0, s, a);
        if (stage < 0 || stage == 2)
            hipLaunchKernelGGL(k_moe_combine, dim3((a.H + TILE_ROWS - 1) / TILE_ROWS), dim3(GEMV_THREADS), 0, s, a);
    }
}

// M > 1: five launches (stage 0: router + plan, 1: gate/up, 2: down + combine)
template <int TE, int TS>
static void launch_layer_multi(const MoeArgs& a, int stage, hipStream_t s) {
    const int NB = a.F / QK, NU = a.M * a.K + 1;
    if (stage < 0 || stage == 0) {
        // four work-groups per router row, two tokens each (M = 8: layer
        // 49.8 -> 49.2 us uniform, 40.9 -> 39.4 us Zipf against one
        // work-group per row; one token each or two rows per work-group
        // measured slower)
        if (a.H == 2048)
            hipLaunchKernelGGL((k_moe_route<MAX_TOK / ROUTE_TS, ROUTE_TS, 2048>), dim3(route_grid(a, ROUTE_TS)), dim3(256),
                               0, s, a);
        else
            hipLaunchKernelGGL((k_moe_route<MAX_TOK / ROUTE_TS, ROUTE_TS>), dim3(route_grid(a, ROUTE_TS)), dim3(256), 0, s,
                               a);
        hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(PLAN_THREADS), 0, s, a);
    }
    if (stage < 0 || stage == 1)
        hipLaunchKernelGGL((k_moe_gateup<TE, TS>), dim3(NB * ((a.has_shared ? (a.M + KG_NT - 1) / KG_NT : 0) + NU - 1)),
                           dim3(GEMV_THREADS), 0, s, a);
    if (stage < 0 || stage == 2) {
        if constexpr (kdc_types<TE, TS>()) {
            if (kdc_fits(a, TE, TS)) {
                hipLaunchKernelGGL((k_moe_down_comb<TE, TS>), dim3(a.H / kdc_rows<TE>()), dim3(KDC_THREADS), 0, s, a);
                return;
            }
        }
        hipLaunchKernelGGL((k_moe_down<TE, TS>), dim3((a.H + 4 * KG_RG - 1) / (4 * KG_RG), NU), dim3(GEMV_THREADS), 0,
                           s, a);
        hipLaunchKernelGGL(k_moe_combine_dn, dim3((a.H + 255) / 256, a.M), dim3(256), 0, s, a);
    }
}

// one token: the fused three-launch layer
template <int TE, int TS>
static void launch_layer(const MoeArgs& a, int stage, hipStream_t s) {
    if constexpr (is_kquant<TS>()) {
        // K-quant shared expert: the one-token kernel where it fits, else the
        // several-token launches (K2 / K3 have no K-quant down path)
        if (a.M == 1 && TS != T_Q6_K && expert1_fits(a, TE, TS))
            launch_layer_nt<TE, TS, 1>(a, stage, s);
        else
            launch_layer_multi<TE, TS>(a, stage, s);
    } else {
        if (a.M == 1) launch_layer_nt<TE, TS, 1>(a, stage, s);
        else launch_layer_multi<TE, TS>(a, stage, s);
    }
}

template <int TE>
static bool dispatch_ts(int ts, const MoeArgs& a, int stage, hipStream_t s) {
    switch (ts) {
    case T_Q8_0: launch_layer<TE, T_Q8_0>(a, stage, s); return true;
    case T_Q4_0: launch_layer<TE, T_Q4_0>(a, stage, s); return true;
    case T_IQ3_S: launch_layer<TE, T_IQ3_S>(a, stage, s); return true;
    case T_Q4_K: launch_layer<TE, T_Q4_K>(a, stage, s); return true;
    case T_Q5_K: launch_layer<TE, T_Q5_K>(a, stage, s); return true;
    case T_Q6_K: launch_layer<TE, T_Q6_K>(a, stage, s); return true;
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
// the shared expert may also be a K-quant (Q5_K in the reference model)
static bool valid_shared_type(int t) { return valid_type(t) || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

// ---------------------------------------------- standalone glue kernels

__global__ __launch_bounds__(256) void k_f32_gemv(const float* A, const float* x, float* y, int cols) {
    __shared__ float red[256];
    float v[1];
    f32_row_dot<1>(A + (int64_t)blockIdx.x * cols, x, cols, 1, red, v);
    if (threadIdx.x == 0) y[blockIdx.x] = v[0];
}

__global__ __launch_bounds__(64) void k_topk(const float* logits, int* idx, float* w, int E, int K) {
    __shared__ uint64_t s_tk[128];
    const int t = blockIdx.x;
    topk_wave_any(logits + (int64_t)t * E, E, K, idx + t * K, w + t * K, s_tk);
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

// ---- no-allocation variant: the workspace is a file-scope device array.
// Each GPU the library runs on holds its own copy (16 MiB) until the process
// ends.  Host code never passes `scratch` itself (in host code the name is a
// stand-in, not a device address): the array's address on each device comes
// from hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t MOE_STATIC_SCRATCH_BYTES = (size_t)16 << 20;
static __device__ __attribute__((aligned(256))) uint8_t scratch[MOE_STATIC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// Device address of this device's scratch (nullptr on failure).
static void* scratch_ptr(int dev) {
    if (dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
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
    CHIMERE_REQUIRE(H > 0 && H % 256 == 0 && H <= 4096 && F > 0 && F % 256 == 0 && F <= 2048, CHIMERE_ERR_ARG,
                    "moe_ffn_decode: hidden=%d (<= 4096) / ffn=%d (<= 2048) must be multiples of 256", H, F);
    CHIMERE_REQUIRE(E >= 1 && E <= MAX_E && K >= 1 && K <= MAX_K && K <= E, CHIMERE_ERR_ARG,
                    "moe_ffn_decode: n_experts=%d top_k=%d out of range", E, K);
    CHIMERE_REQUIRE(valid_type(L->expert_type), CHIMERE_ERR_ARG, "moe_ffn_decode: expert_type %d", L->expert_type);
    const bool has_sh = L->shared_type >= 0;
    CHIMERE_REQUIRE(!has_sh || (valid_shared_type(L->shared_type) && L->sh_gate && L->sh_up && L->sh_down),
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
    a.xq = w + p.xq; a.terms = (uint2*)(w + p.terms); a.lane_acc = (float*)(w + p.terms);
    a.xq_stride = p.xq_stride;
    a.hq = w + p.hq; a.dn = (float*)(w + p.terms); a.hq_stride = p.hq_stride;
    dispatch_layer(L->expert_type, L->shared_type, a, stage, stream);
    check_launch("moe_ffn_decode");
}

void chimere_moe_ffn_decode(const chimere_moe_layer* L, const float* x, float* out, int ntok,
                            int* ids_out, float* w_out, void* workspace, size_t ws_bytes,
                            hipStream_t stream) {
    moe_decode(L, x, out, ntok, ids_out, w_out, workspace, ws_bytes, -1, stream);
}

void chimere_moe_ffn_decode_noalloc(const chimere_moe_layer* L, const float* x, float* out, int ntok,
                                    int* ids_out, float* w_out, hipStream_t stream) {
    CHIMERE_REQUIRE(L, CHIMERE_ERR_ARG, "moe_ffn_decode_noalloc: null layer");
    CHIMERE_REQUIRE(ntok >= 1 && ntok <= MAX_TOK, CHIMERE_ERR_ARG, "moe_ffn_decode_noalloc: ntok=%d not in 1..8",
                    ntok);
    const size_t need = chimere_moe_workspace_size(L, ntok);
    CHIMERE_REQUIRE(need > 0, CHIMERE_ERR_ARG, "moe_ffn_decode_noalloc: layer shape rejected");
    CHIMERE_REQUIRE(need <= MOE_STATIC_SCRATCH_BYTES, CHIMERE_ERR_WORKSPACE,
                    "moe_ffn_decode_noalloc: layer needs %zu scratch bytes > the static %zu", need,
                    MOE_STATIC_SCRATCH_BYTES);
    int dev = -1;
    CHIMERE_REQUIRE(hipGetDevice(&dev) == hipSuccess, CHIMERE_ERR_LAUNCH, "moe_ffn_decode_noalloc: no device");
    void* ws = scratch_ptr(dev);
    CHIMERE_REQUIRE(ws, CHIMERE_ERR_LAUNCH, "moe_ffn_decode_noalloc: hipGetSymbolAddress failed on device %d", dev);
    moe_decode(L, x, out, ntok, ids_out, w_out, ws, MOE_STATIC_SCRATCH_BYTES, -1, stream);
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
