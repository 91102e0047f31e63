// fused_moe.hip -- the expert FFN on unquantized (f32) activations with IQ3_S
// weights: the reference's fused_moe_iq3s (cs/src/kernels/fused_moe.rs:261-468,
// cs/kernels/chimere_kernels.cu:1093-1143), its GPU expert path when the
// ggml Q8_1 kernels are not selected (cs/src/qwen35_model/moe_ffn.rs:1476-1500).
//
//   for each selected expert k:  g = G_e x,  u = U_e x  (f32 x)
//                                h = silu(g) * u
//                                y_k = D_e h
//   output += sum_k w_k * y_k
//
// The reference runs one block per expert and adds w_k * y_k into output with
// atomicAdd (an order that varies between runs).  Here two launches, and a
// fixed fp32 order:
//   * a row's dot: lane j of its 16-lane group takes the 32-element blocks
//     j, j+16, ... in ascending order; a block's sum is s = fmaf(level_e, x_e, s)
//     over its 32 elements (signed int8 levels, exact as f32), then
//     acc = fmaf(f32(d) * (1 + 2 * scale), s, acc); the 16 lanes are summed by
//     the halving tree xor 8, 4, 2, 1;
//   * h = det_silu(g) * u;
//   * output[r] = output[r] + a, a = fmaf(w_k, y_k[r], a) over k ascending from 0.
// Launch 1 (gate/up): grid (F/32, K), 1024 threads: gate rows [32w, 32w+32) and
// the same up rows of expert ids[k] (64 rows, one per 16-lane group), the
// activation row in LDS, weight rows staged in 64-block chunks; h to the
// workspace.  Launch 2 (down + combine): grid H/8, 128 threads: 8 down rows
// for every expert (all K experts' row runs staged at once), then the combine.
#include "api_internal.h"
#include "common.h"

namespace chimere {

__constant__ uint32_t c_iq3s_grid_fm[512] = CHIMERE_IQ3S_GRID_INIT;

constexpr int FM_RG = 64;                   // gate/up rows per work-group (32 gate + 32 up)
constexpr int FM_THREADS = FM_RG * SLOTS;   // 1024
constexpr int FM_CBLK = 64;                 // 32-element blocks per staged chunk (8 superblocks)
constexpr int FM_CB = FM_CBLK / 8 * 110;    // 880 bytes of a row per chunk
constexpr int FM_MAX_H = 4096;              // activation row in LDS (16 KiB)
constexpr int FM_DR = 8;                    // down rows per work-group
constexpr int FM_MAX_F = 512;               // down rows staged whole: F / 256 superblocks
constexpr int FM_MAX_K = 16;

struct FmArgs {
    const float* x;
    const uint8_t *gate, *up, *down;
    const int* ids;
    const float* wts;
    float* out;
    float* h;   // [K][F] workspace
    int H, F, K;
    int64_t bg, bu, bd;   // bytes per expert
};

// s = fmaf(level_e, x_e, s) over the block's 32 elements in order
__device__ __forceinline__ float blk_dot_f32(const WBlk& w, const float* __restrict__ xb) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
        for (int i = 0; i < 4; i++) s = __builtin_fmaf((float)(int)(int8_t)(w.v[k] >> (8 * i)), xb[4 * k + i], s);
    return s;
}

__global__ __launch_bounds__(FM_THREADS) void k_fm_gate_up(FmArgs a) {
    __shared__ float xs[FM_MAX_H];
    __shared__ __attribute__((aligned(16))) uint8_t tile[FM_RG * FM_CB + 16];
    __shared__ uint32_t grid[512];
    __shared__ float hg[QK], hu[QK];
    const int tid = threadIdx.x, g = tid >> 4, j = tid & 15;
    const int w = blockIdx.x, k = blockIdx.y;
    const int64_t e = a.ids[k];
    const int nb = a.H / QK;
    const int64_t rb = (int64_t)a.H / 256 * 110;
    for (int i = tid; i < a.H; i += FM_THREADS) xs[i] = a.x[i];
    for (int i = tid; i < 512; i += FM_THREADS) grid[i] = c_iq3s_grid_fm[i];
    const uint8_t* g0 = a.gate + e * a.bg + (int64_t)w * QK * rb;
    const uint8_t* u0 = a.up + e * a.bu + (int64_t)w * QK * rb;
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += FM_CBLK) {
        const int cb = min(FM_CBLK, nb - b0), seg = cb / 8 * 110;
        const int64_t goff = (int64_t)b0 / 8 * 110;
        __syncthreads();   // the previous chunk is consumed (and xs / grid written)
        stage_rows<true, CPOL_STREAM>(tile, g0 + goff, rb, QK, seg, tid, FM_THREADS);
        stage_rows<true, CPOL_STREAM>(tile + QK * seg, u0 + goff, rb, QK, seg, tid, FM_THREADS);
        lds_copy_wait();
        __syncthreads();
        const uint8_t* row = tile + g * seg;
        for (int b = j; b < cb; b += SLOTS) {
            WBlk wb;
            block_decode<T_IQ3_S>(row, b, grid, wb);
            const float s = blk_dot_f32(wb, xs + QK * (b0 + b));
            acc = __builtin_fmaf(wb.dw * (float)wb.mult, s, acc);
        }
    }
    const float v = slot_reduce16(acc);
    if (j == 0) {
        if (g < QK) hg[g] = v;
        else hu[g - QK] = v;
    }
    __syncthreads();
    if (tid < QK) a.h[(int64_t)k * a.F + w * QK + tid] = det_silu(hg[tid]) * hu[tid];
}

__global__ __launch_bounds__(FM_DR * SLOTS) void k_fm_down(FmArgs a) {
    constexpr int RUN = FM_DR * (FM_MAX_F / 256 * 110);   // bytes of one expert's FM_DR rows at most
    __shared__ __attribute__((aligned(16))) uint8_t wl[FM_MAX_K * RUN + 16];
    __shared__ uint32_t grid[512];
    const int tid = threadIdx.x, g = tid >> 4, j = tid & 15;
    const int r0 = blockIdx.x * FM_DR;
    const int nb = a.F / QK;
    const int64_t rb = (int64_t)a.F / 256 * 110;
    const int run = FM_DR * (int)rb;
    for (int i = tid; i < 512; i += FM_DR * SLOTS) grid[i] = c_iq3s_grid_fm[i];
    for (int k = 0; k < a.K; k++)
        stage_rows<true, CPOL_STREAM>(wl + k * run, a.down + (int64_t)a.ids[k] * a.bd + r0 * rb, rb, FM_DR,
                                      (int)rb, tid, FM_DR * SLOTS);
    lds_copy_wait();
    __syncthreads();
    float o = 0.0f;
    for (int k = 0; k < a.K; k++) {
        const uint8_t* row = wl + k * run + g * rb;
        const float* hk = a.h + (int64_t)k * a.F;
        float acc = 0.0f;
        for (int b = j; b < nb; b += SLOTS) {
            WBlk wb;
            block_decode<T_IQ3_S>(row, b, grid, wb);
            float hb[QK];
#pragma unroll
            for (int i = 0; i < QK / 4; i++) *(float4*)(hb + 4 * i) = *(const float4*)(hk + QK * b + 4 * i);
            acc = __builtin_fmaf(wb.dw * (float)wb.mult, blk_dot_f32(wb, hb), acc);
        }
        o = __builtin_fmaf(a.wts[k], slot_reduce16(acc), o);
    }
    if (j == 0) a.out[r0 + g] = a.out[r0 + g] + o;
}

}  // namespace chimere

using namespace chimere;

extern "C" {

size_t chimere_fused_moe_iq3s_workspace_size(int hidden_size, int expert_ffn, int top_k) {
    (void)hidden_size;
    if (expert_ffn <= 0 || top_k <= 0) return 0;
    return (size_t)top_k * expert_ffn * sizeof(float);
}

void chimere_fused_moe_iq3s(const float* hidden, const void* gate_exps, const void* up_exps, const void* down_exps,
                            const int* expert_ids, const float* expert_weights, float* output, int hidden_size,
                            int expert_ffn, int64_t expert_bytes_gate, int64_t expert_bytes_up,
                            int64_t expert_bytes_down, int top_k, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    CHIMERE_REQUIRE(hidden && gate_exps && up_exps && down_exps && expert_ids && expert_weights && output &&
                        workspace,
                    CHIMERE_ERR_ARG, "fused_moe_iq3s: null pointer");
    const int H = hidden_size, F = expert_ffn, K = top_k;
    CHIMERE_REQUIRE(H >= 256 && H % 256 == 0 && H <= FM_MAX_H && F >= 256 && F % 256 == 0 && F <= FM_MAX_F,
                    CHIMERE_ERR_ARG,
                    "fused_moe_iq3s: hidden_size=%d (multiple of 256, <= %d), expert_ffn=%d (multiple of 256, <= %d)",
                    H, FM_MAX_H, F, FM_MAX_F);
    CHIMERE_REQUIRE(K >= 1 && K <= FM_MAX_K, CHIMERE_ERR_ARG, "fused_moe_iq3s: top_k=%d (1..%d)", K, FM_MAX_K);
    const int64_t rbH = (int64_t)H / 256 * 110, rbF = (int64_t)F / 256 * 110;
    CHIMERE_REQUIRE(expert_bytes_gate >= rbH * F && expert_bytes_up >= rbH * F && expert_bytes_down >= rbF * H,
                    CHIMERE_ERR_ARG, "fused_moe_iq3s: expert byte strides too small");
    CHIMERE_REQUIRE((((uintptr_t)gate_exps | (uintptr_t)up_exps | (uintptr_t)down_exps | (uintptr_t)expert_bytes_gate |
                      (uintptr_t)expert_bytes_up | (uintptr_t)expert_bytes_down) & 3) == 0 &&
                        ((uintptr_t)hidden & 15) == 0,
                    CHIMERE_ERR_ARG, "fused_moe_iq3s: weights must be 4-byte aligned, hidden 16-byte aligned");
    CHIMERE_REQUIRE(workspace_bytes >= chimere_fused_moe_iq3s_workspace_size(H, F, K) &&
                        ((uintptr_t)workspace & 15) == 0,
                    CHIMERE_ERR_WORKSPACE, "fused_moe_iq3s: workspace %zu bytes < %zu (or not 16-byte aligned)",
                    workspace_bytes, chimere_fused_moe_iq3s_workspace_size(H, F, K));
    FmArgs a{};
    a.x = hidden;
    a.gate = (const uint8_t*)gate_exps; a.up = (const uint8_t*)up_exps; a.down = (const uint8_t*)down_exps;
    a.ids = expert_ids; a.wts = expert_weights; a.out = output; a.h = (float*)workspace;
    a.H = H; a.F = F; a.K = K;
    a.bg = expert_bytes_gate; a.bu = expert_bytes_up; a.bd = expert_bytes_down;
    hipLaunchKernelGGL(k_fm_gate_up, dim3(F / QK, K), dim3(FM_THREADS), 0, stream, a);
    hipLaunchKernelGGL(k_fm_down, dim3(H / FM_DR), dim3(FM_DR * SLOTS), 0, stream, a);
    check_launch("fused_moe_iq3s");
}

}  // extern "C"
