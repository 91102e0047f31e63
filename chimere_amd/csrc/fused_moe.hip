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
//   * a row's dot over L lanes (gate / up rows: L = 64, one wave per row; down
//     rows: L = 16): lane j takes the 32-element blocks j, j+L, ... in
//     ascending order; a block's sum is s = fmaf(level_e, x_e, s) over its 32
//     elements (signed int8 levels, exact as f32), then
//     acc = fmaf(f32(d) * (1 + 2 * scale), s, acc); the L lanes are summed by
//     the halving tree (lanes j, j + m for m = L/2, ..., 1);
//   * h = det_silu(g) * u;
//   * output[r] = output[r] + a, a = fmaf(w_k, y_k[r], a) over k ascending from 0.
// Launch 1 (gate/up): grid (F/2, K), 256 threads: gate rows 2w, 2w+1 and the
// same up rows of expert ids[k] (one wave each; h needs only a row's own gate
// and up values), the activation row in LDS, weight rows staged in 64-block
// chunks (one block per lane per chunk); h to the workspace.  Launch 2 (down + combine):
// grid ceil(H/R), 256 threads, R = 16 / K rows: 16-lane group g takes down row
// r0 + g / K of expert g % K; the R rows' K results are then combined in k
// order by one thread per row.
#include "api_internal.h"
#include "common.h"

namespace chimere {

__constant__ uint32_t c_iq3s_grid_fm[512] = CHIMERE_IQ3S_GRID_INIT;

// gate rows per work-group (and as many up rows): 2 (2048 work-groups of 4
// waves for F = 512, top-8) measured 10.3 us against 12.3 us with 8
constexpr int FM_GR = 2;
constexpr int FM_THREADS = 2 * FM_GR * 64;   // a wave per gate / up row
constexpr int FM_CBLK = 64;                 // 32-element blocks per staged chunk (8 superblocks)
constexpr int FM_CB = FM_CBLK / 8 * 110;    // 880 bytes of a row per chunk
constexpr int FM_MAX_H = 4096;              // activation row in LDS (16 KiB)
constexpr int FM_MAX_F = 512;               // a down row staged whole: F / 256 superblocks
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

// HC / FC: H and F as compile-time constants (0: the run-time a.H / a.F)
template <int HC = 0, int FC = 0>
__global__ __launch_bounds__(FM_THREADS) void k_fm_gate_up(FmArgs a) {
    const int H = HC ? HC : a.H, F = FC ? FC : a.F;
    __shared__ __attribute__((aligned(16))) float xs[FM_MAX_H];
    __shared__ __attribute__((aligned(16))) uint8_t tile[2 * FM_GR * FM_CB + 16];
    __shared__ uint32_t grid[512];
    __shared__ float hg[FM_GR], hu[FM_GR];
    const int tid = threadIdx.x, g = tid >> 6, j = tid & 63;
    const int w = blockIdx.x, k = blockIdx.y;
    const int64_t e = a.ids[k];
    const int nb = H / QK;
    const int64_t rb = (int64_t)H / 256 * 110;
    const uint8_t* g0 = a.gate + e * a.bg + (int64_t)w * FM_GR * rb;
    const uint8_t* u0 = a.up + e * a.bu + (int64_t)w * FM_GR * rb;
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += FM_CBLK) {
        const int cb = min(FM_CBLK, nb - b0), seg = cb / 8 * 110;
        const int64_t goff = (int64_t)b0 / 8 * 110;
        if (b0) __syncthreads();   // the previous chunk is consumed
        stage_rows<true, CPOL_STREAM>(tile, g0 + goff, rb, FM_GR, seg, tid, FM_THREADS);
        stage_rows<true, CPOL_STREAM>(tile + FM_GR * seg, u0 + goff, rb, FM_GR, seg, tid, FM_THREADS);
        if (b0 == 0) {   // the activation row and the codebook, while the first chunk's rows are in flight
            for (int i = tid; i < H / 4; i += FM_THREADS) ((float4*)xs)[i] = ((const float4*)a.x)[i];
            for (int i = tid; i < 512; i += FM_THREADS) grid[i] = c_iq3s_grid_fm[i];
        }
        lds_copy_wait();
        __syncthreads();
        const uint8_t* row = tile + g * seg;
        if (j < cb) {   // chunks of 64 blocks: block j
            WBlk wb;
            block_decode<T_IQ3_S>(row, j, grid, wb);
            const float s = blk_dot_f32(wb, xs + QK * (b0 + j));
            acc = __builtin_fmaf(wb.dw * (float)wb.mult, s, acc);
        }
    }
    // the 64 lanes by the halving tree (lane 0 holds it)
    float v = acc + xlane<32>(acc);
    v = v + xlane<16>(v);
    v = slot_reduce16(v);
    if (j == 0) {
        if (g < FM_GR) hg[g] = v;
        else hu[g - FM_GR] = v;
    }
    __syncthreads();
    if (tid < FM_GR) a.h[(int64_t)k * F + w * FM_GR + tid] = det_silu(hg[tid]) * hu[tid];
}

template <int HC = 0, int FC = 0>
__global__ __launch_bounds__(256) void k_fm_down(FmArgs a) {
    const int H = HC ? HC : a.H, F = FC ? FC : a.F;
    constexpr int ROWB = FM_MAX_F / 256 * 110;   // bytes of a down row at most
    __shared__ __attribute__((aligned(16))) uint8_t wl[16 * ROWB + 16];
    __shared__ uint32_t grid[512];
    __shared__ float ys[16];
    __shared__ int s_ids[FM_MAX_K];
    __shared__ float s_w[FM_MAX_K];
    const int tid = threadIdx.x, g = tid >> 4, j = tid & 15;
    const int K = a.K, R = 16 / K, r0 = blockIdx.x * R;
    const int nb = F / QK;
    const int rb = F / 256 * 110;
    if (tid < K) {
        s_ids[tid] = a.ids[tid];
        s_w[tid] = a.wts[tid];
    }
    for (int i = tid; i < 512; i += 256) grid[i] = c_iq3s_grid_fm[i];
    // group g: down row r0 + g / K of expert g % K
    const bool act = g < R * K && r0 + g / K < H;
    const int k = g % K;
    // prefetched while the ids load: this lane's h block (F <= 512: block j
    // only) and the output values of the combining threads
    float hb[QK];
    if (act && j < nb) {
        const float* hk = a.h + (int64_t)k * F + QK * j;
#pragma unroll
        for (int i = 0; i < QK / 4; i++) *(float4*)(hb + 4 * i) = *(const float4*)(hk + 4 * i);
    }
    const bool comb = tid < R && r0 + tid < H;
    const float out0 = comb ? a.out[r0 + tid] : 0.0f;
    __syncthreads();   // s_ids, s_w, grid
    if (act) {
        // the group stages its own row (lanes of one wave: visible to the
        // group once its LDS writes are done)
        uint8_t* row = wl + g * ROWB;
        const uint8_t* src = a.down + (int64_t)s_ids[k] * a.bd + (int64_t)(r0 + g / K) * rb;
        if ((rb & 3) == 0) {
            for (int c = j; c < rb / 4; c += SLOTS) ((uint32_t*)row)[c] = ((const uint32_t*)src)[c];
        } else {
            for (int c = j; c < rb / 2; c += SLOTS) ((uint16_t*)row)[c] = ((const uint16_t*)src)[c];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        float acc = 0.0f;
        if (j < nb) {   // F <= 512: one block per lane
            WBlk wb;
            block_decode<T_IQ3_S>(row, j, grid, wb);
            acc = __builtin_fmaf(wb.dw * (float)wb.mult, blk_dot_f32(wb, hb), acc);
        }
        const float v = slot_reduce16(acc);
        if (j == 0) ys[g] = v;
    }
    __syncthreads();
    if (comb) {
        float o = 0.0f;
        for (int kk = 0; kk < K; kk++) o = __builtin_fmaf(s_w[kk], ys[tid * K + kk], o);
        a.out[r0 + tid] = out0 + o;
    }
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
    const int R = 16 / K;
    if (H == 2048 && F == 512) {
        hipLaunchKernelGGL((k_fm_gate_up<2048, 512>), dim3(F / FM_GR, K), dim3(FM_THREADS), 0, stream, a);
        hipLaunchKernelGGL((k_fm_down<2048, 512>), dim3((H + R - 1) / R), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_fm_gate_up<>), dim3(F / FM_GR, K), dim3(FM_THREADS), 0, stream, a);
        hipLaunchKernelGGL((k_fm_down<>), dim3((H + R - 1) / R), dim3(256), 0, stream, a);
    }
    check_launch("fused_moe_iq3s");
}

}  // extern "C"
