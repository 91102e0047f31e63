/*
 * chimere_hip.h -- C ABI of libchimere_hip.so, the MI355X (gfx950) decode-time
 * quantized GEMV / MoE-FFN path.
 *
 * Drop-in for the reference's extern "C" boundary
 *   chimere-server/ffi/ggml_cuda_gemv.cu:94-463
 * as declared on the Rust side in
 *   chimere-server/src/kernels/ggml_gpu.rs:101-240.
 * Names, argument order and meaning of the mirrored entry points are the
 * reference's; cudaStream_t becomes hipStream_t (an opaque pointer; NULL is
 * the default stream).  Every pointer argument is a caller-owned DEVICE
 * pointer unless stated otherwise; outputs are overwritten.  No entry point
 * allocates, frees or synchronizes, so all of them may be recorded into a
 * HIP graph.  Entry points return void like the reference's; a rejected
 * argument or a failed launch is reported by chimere_hip_get_last_error().
 *
 * Block formats (byte-exact with ggml): Q8_0 34 B / 32, Q4_0 18 B / 32,
 * Q8_1 36 B / 32 ([f16 d][f16 s = sum x][i8 q[32]]), IQ3_S 110 B / 256.
 * Type ids below follow ggml's enum.
 */
#ifndef CHIMERE_HIP_H
#define CHIMERE_HIP_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHIMERE_TYPE_Q4_0 2
#define CHIMERE_TYPE_Q8_0 8
#define CHIMERE_TYPE_IQ3_S 21

/* error codes returned by chimere_hip_get_last_error() */
#define CHIMERE_OK 0
#define CHIMERE_ERR_ARG 1      /* rejected argument (shape, alignment, null, range) */
#define CHIMERE_ERR_LAUNCH 2   /* kernel launch failed */
#define CHIMERE_ERR_WORKSPACE 3/* workspace too small */

/* ---------------------------------------------------------------- sizes */
/* ggml_cuda_gemv.cu:197-209 */
int chimere_q8_1_block_bytes(void);   /* 36 */
int chimere_q8_1_block_elems(void);   /* 32 */
int chimere_matrix_row_padding(void); /* 512 */

/* ----------------------------------------------------- activation quant */
/* ggml_cuda_gemv.cu:184-194.  input f32[ncols] -> Q8_1 blocks; out holds
 * ncols_padded/32 blocks (elements ncols..ncols_padded-1 quantize as 0). */
void chimere_quantize_q8_1(const float *input, void *output, int64_t ncols,
                           int64_t ncols_padded, hipStream_t stream);
/* ggml_cuda_gemv.cu:393-404.  batch rows of ncols (input row stride ncols);
 * output row stride ncols_padded/32*36 bytes. */
void chimere_quantize_q8_1_batched(const float *input, void *output, int64_t ncols,
                                   int64_t ncols_padded, int batch, hipStream_t stream);

/* --------------------------------------------------------------- GEMV */
/* y[r] = W[r,:] . x for W [nrows, ncols] quantized, x Q8_1 with
 * nrows_y_padded (= pad(ncols,512)/32) blocks.  ggml_cuda_gemv.cu:105-116
 * (iq3s), :133-144 (q8_0); Q4_0 has no counterpart in the reference's ABI
 * (ggml mul_mat_vec_q4_0_q8_1 is reached there only through libllama) and is
 * added with the same signature. */
void chimere_mmvq_iq3s(const void *weights, const void *input_q8, float *output,
                       int ncols, int nrows, int nrows_y_padded, hipStream_t stream);
void chimere_mmvq_q8_0(const void *weights, const void *input_q8, float *output,
                       int ncols, int nrows, int nrows_y_padded, hipStream_t stream);
void chimere_mmvq_q4_0(const void *weights, const void *input_q8, float *output,
                       int ncols, int nrows, int nrows_y_padded, hipStream_t stream);

/* The same Q4_0 GEMV with ggml's block term (mul_mat_vec_q4_0_q8_1, reached
 * in the reference only through libllama, out of tree): per block
 * d_w * (sum(nib * q_x) * d_x - 8 * s_x), s_x = the Q8_1 block's f16 sum of
 * x, contracted as inner = fmaf(sum, d_x, -8 s_x), acc = fmaf(d_w, inner,
 * acc).  For ggml-parity experiments: it differs from chimere_mmvq_q4_0's
 * exact integer form by at most 8 |d_w| |s_x - d_x * sum(q_x)| per block plus
 * fp32 rounding.  Block terms are combined in this library's order (16 lanes
 * per row, halving tree); ggml's own split of a block over threads is not
 * reproduced. */
void chimere_mmvq_q4_0_sform(const void *weights, const void *input_q8, float *output,
                             int ncols, int nrows, int nrows_y_padded, hipStream_t stream);

/* Fused F32 -> Q8_1 -> GEMV (ggml_cuda_gemv.cu:302-387): quantizes input_f32
 * into q8_scratch (pad(ncols,512)/32*36 bytes) then runs the GEMV. */
void chimere_mmvq_iq3s_f32(const void *weights, const float *input_f32, float *output,
                           int ncols, int nrows, int ncols_padded, void *q8_scratch,
                           hipStream_t stream);
void chimere_mmvq_q8_0_f32(const void *weights, const float *input_f32, float *output,
                           int ncols, int nrows, int ncols_padded, void *q8_scratch,
                           hipStream_t stream);
void chimere_mmvq_q4_0_f32(const void *weights, const float *input_f32, float *output,
                           int ncols, int nrows, int ncols_padded, void *q8_scratch,
                           hipStream_t stream);

/* ggml K-quant and MXFP4 weights (ggml_cuda_gemv.cu:118-175, 292-387, 407-460).
 * Block layouts: Q4_K 144 B / 256 (f16 d, f16 dmin, 12 packed 6-bit
 * scale/min bytes, qs[128]; gguf_loader.rs:1265-1330), Q5_K 176 B / 256 (+
 * qh[32] high bits; gguf_loader.rs:1165-1263), Q6_K 210 B / 256 (ql[128],
 * qh[64], int8 scales[16], f16 d; gguf_loader.rs:839-917), MXFP4 17 B / 32
 * (E8M0 scale byte, 16 bytes of E2M1 nibbles, low nibble = element j, high =
 * j+16).  Per 32-element block: sumi exact in int32; Q4_K / Q5_K add the min
 * term -f32(dmin)*f32(d_x) * (m * sum q_x) as a second fmaf in the same order. */
void chimere_mmvq_q5k(const void *weights, const void *input_q8, float *output,
                      int ncols, int nrows, int nrows_y_padded, hipStream_t stream);
void chimere_mmvq_q4k(const void *weights, const void *input_q8, float *output,
                      int ncols, int nrows, int nrows_y_padded, hipStream_t stream);
void chimere_mmvq_q6k(const void *weights, const void *input_q8, float *output,
                      int ncols, int nrows, int nrows_y_padded, hipStream_t stream);
void chimere_mmvq_mxfp4(const void *weights, const void *input_q8, float *output,
                        int ncols, int nrows, int nrows_y_padded, hipStream_t stream);
void chimere_mmvq_q5k_f32(const void *weights, const float *input_f32, float *output,
                          int ncols, int nrows, int ncols_padded, void *q8_scratch,
                          hipStream_t stream);
void chimere_mmvq_q4k_f32(const void *weights, const float *input_f32, float *output,
                          int ncols, int nrows, int ncols_padded, void *q8_scratch,
                          hipStream_t stream);
void chimere_mmvq_q6k_f32(const void *weights, const float *input_f32, float *output,
                          int ncols, int nrows, int ncols_padded, void *q8_scratch,
                          hipStream_t stream);
/* ggml_cuda_gemv.cu:448-461: note the argument order (scratch before output). */
void chimere_mmvq_mxfp4_f32(const void *weights, const float *input_f32, void *q8_scratch,
                            float *output, int ncols, int nrows, int ncols_padded,
                            hipStream_t stream);
/* ggml_cuda_gemv.cu:425-445, same contract as chimere_mmvq_iq3s_batched below:
 * expert_ids is a DEVICE array (the reference reads it on the host). */
void chimere_mmvq_mxfp4_batched(const void *all_weights, const void *input_q8, float *output,
                                const int *expert_ids, int ncols, int nrows, int nrows_y_padded,
                                int64_t expert_stride, int64_t input_stride, int top_k,
                                hipStream_t stream);

/* Batched expert GEMV with device-resident expert ids (ggml_cuda_gemv.cu:243-279):
 * for k < top_k: output[k*nrows + r] = W_{ids[k]}[r,:] . x_k with
 * W_e = all_weights + e*expert_stride bytes and x_k = input_q8 + k*input_stride
 * bytes (input_stride 0 = one shared input).  The q8_0 / q4_0 variants are
 * additions with the same signature. */
void chimere_mmvq_iq3s_batched(const void *all_weights, const void *input_q8, float *output,
                               const int *expert_ids, int ncols, int nrows, int nrows_y_padded,
                               int64_t expert_stride, int64_t input_stride, int top_k,
                               hipStream_t stream);
void chimere_mmvq_q8_0_batched(const void *all_weights, const void *input_q8, float *output,
                               const int *expert_ids, int ncols, int nrows, int nrows_y_padded,
                               int64_t expert_stride, int64_t input_stride, int top_k,
                               hipStream_t stream);
void chimere_mmvq_q4_0_batched(const void *all_weights, const void *input_q8, float *output,
                               const int *expert_ids, int ncols, int nrows, int nrows_y_padded,
                               int64_t expert_stride, int64_t input_stride, int top_k,
                               hipStream_t stream);

/* Multi-token dense GEMV (M <= 8 concurrent decode tokens; no reference
 * counterpart -- the reference runs one token at a time): token t's Q8_1
 * input at input_q8 + t*nrows_y_padded*36, output[t*nrows + r]. */
void chimere_mmvq_multi(int type, const void *weights, const void *input_q8, float *output,
                        int ncols, int nrows, int nrows_y_padded, int ntok, hipStream_t stream);
/* The same per weight type (the per-type names of the boundary's additions). */
void chimere_mmvq_q4_0_multi(const void *weights, const void *input_q8, float *output, int ncols,
                             int nrows, int nrows_y_padded, int ntok, hipStream_t stream);
void chimere_mmvq_q8_0_multi(const void *weights, const void *input_q8, float *output, int ncols,
                             int nrows, int nrows_y_padded, int ntok, hipStream_t stream);
void chimere_mmvq_iq3s_multi(const void *weights, const void *input_q8, float *output, int ncols,
                             int nrows, int nrows_y_padded, int ntok, hipStream_t stream);

/* ------------------------------------------------------- routing / glue */
/* f32 GEMV, y[r] = sum_c A[r*cols+c] x[c]  (src/kernels/elementwise.rs:186-221,
 * raw_f32_gemv :599-629); same 256-lane strided order and halving tree. */
void chimere_f32_gemv(const float *A, const float *x, float *y, int rows, int cols,
                      hipStream_t stream);
/* softmax over n_experts logits, top-k by probability (ties -> lowest index),
 * renormalised weights (kernels/chimere_kernels.cu:1150-1223,
 * src/kernels/topk_softmax.rs:113).  ntok rows of logits (row stride
 * n_experts); idx/w rows of top_k.  n_experts <= 1024. */
void chimere_topk_softmax(const float *logits, int *top_idx, float *top_w, int n_experts,
                          int top_k, int ntok, hipStream_t stream);
/* gate[i] = silu(gate[i]) * up[i]   (src/kernels/fused_ops.rs:34-45) */
void chimere_silu_mul_inplace(float *gate, const float *up, int n, hipStream_t stream);
/* acc[h] = sum_k w[k] * expert_outs[k*hidden + h], k ascending
 * (src/kernels/fused_ops.rs:364-378) */
void chimere_weighted_combine(const float *expert_outs, const float *weights, float *acc,
                              int hidden, int top_k, hipStream_t stream);
/* out[i] = out[i] * sigmoid(gate[0]) + combined[i]  (src/scratch_pool.rs:264-277) */
void chimere_sigmoid_gate_add(float *out, const float *gate_logit, const float *combined,
                              int n, hipStream_t stream);

/* ------------------------------------------------------ fused MoE layer */
/* One routed MoE FFN layer (src/qwen35_model/moe_ffn.rs:1081-1768, V3
 * batched path + shared expert): router f32 GEMV (+ optional per-expert
 * logit bias) -> softmax/top-k/renorm -> Q8_1(x) -> gate/up GEMV of each
 * selected expert -> silu(gate)*up -> Q8_1 -> down GEMV -> router-weighted
 * sum (k ascending) -> + shared expert (times sigmoid(<x, sh_gate_w>) when
 * sh_gate_w is non-NULL).  ntok <= 8 tokens route independently; each
 * distinct selected expert's weights are streamed once per call. */
typedef struct chimere_moe_layer {
    int hidden;            /* H, multiple of 256 */
    int ffn;               /* F, multiple of 256 (expert intermediate size) */
    int n_experts;         /* E <= 1024 */
    int top_k;             /* K <= 16 */
    int expert_type;       /* CHIMERE_TYPE_* of gate/up/down experts */
    int shared_type;       /* CHIMERE_TYPE_* of the shared expert, or -1 for none */
    const float *router_w; /* [E, H] f32 row-major */
    const float *logit_bias; /* [E] added to router logits, or NULL */
    const void *gate_exps; /* [E] x [F rows of H] */
    const void *up_exps;   /* [E] x [F rows of H] */
    const void *down_exps; /* [E] x [H rows of F] */
    int64_t gate_stride, up_stride, down_stride; /* bytes per expert */
    const void *sh_gate, *sh_up, *sh_down;       /* shared expert, [F,H] [F,H] [H,F] */
    const float *sh_gate_w;  /* [H] shared-expert gate vector or NULL (gate = 1) */
} chimere_moe_layer;

/* Workspace bytes for chimere_moe_ffn_decode at up to max_ntok tokens. */
size_t chimere_moe_workspace_size(const chimere_moe_layer *layer, int max_ntok);
/* Clears a workspace (a fill kernel, graph-safe).  Optional: the decode
 * kernels keep no counters or flags in the workspace, and every field a call
 * reads was written earlier in the same call, so a workspace is reused across
 * calls without clearing.  Calls sharing one workspace must not overlap. */
void chimere_moe_workspace_init(void *workspace, size_t bytes, hipStream_t stream);
/* x [ntok, H] f32 -> out [ntok, H] f32.  ids_out [ntok, K] / w_out [ntok, K]
 * receive the routing when non-NULL. */
void chimere_moe_ffn_decode(const chimere_moe_layer *layer, const float *x, float *out,
                            int ntok, int *ids_out, float *w_out, void *workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* No-allocation variant of chimere_moe_ffn_decode (no counterpart in the
 * reference): for callers that cannot allocate -- code under HIP-graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments and results without the workspace: the scratch is a static
 * 16 MiB device array per GPU (enough for H <= 2048, F <= 512, E <= 256,
 * top-8 at 8 tokens); larger layers are rejected with CHIMERE_ERR_WORKSPACE.
 * Nothing is allocated or freed; no scratch field needs clearing (every call
 * writes what it reads).  Calls that overlap on one GPU (other streams, other
 * host threads) share that scratch and race: serialise them. */
void chimere_moe_ffn_decode_noalloc(const chimere_moe_layer *layer, const float *x, float *out,
                                    int ntok, int *ids_out, float *w_out, hipStream_t stream);

/* Profiling variant (no reference counterpart): launches only kernel `stage`
 * of chimere_moe_ffn_decode (0 router/top-k, 1 gate/up + SiLU, 2 down +
 * combine; -1 all) on a workspace that a full call with the same layer, x and
 * ntok has prepared; used to time each kernel on its own. */
void chimere_moe_ffn_decode_stage(const chimere_moe_layer *layer, const float *x, float *out,
                                  int ntok, void *workspace, size_t workspace_bytes, int stage,
                                  hipStream_t stream);

/* Routed MoE layer for a chunk of ntok >= 1 tokens (prompt prefill).
 * Replaces the reference's per-token loop over the decode MoE during prefill
 * (src/qwen35_model/compute_graph.rs:1787-1800, moe_ffn.rs:1081-1768 per
 * token): tokens are grouped by expert and the expert projections run as int8
 * matrix-core GEMMs.  Same routing and arithmetic per token as
 * chimere_moe_ffn_decode except the fp32 accumulation order of the quantized
 * projections, which is ascending block order (one accumulator per row).
 * Q4_0 / Q8_0 / IQ3_S experts; the shared expert also Q4_K / Q5_K / Q6_K (the
 * reference model's Q5_K, compute_graph.rs:997-999).  ids_out / w_out (both or
 * neither) receive [ntok][top_k].  No allocation; workspace from
 * chimere_moe_prefill_workspace_size(layer, >= ntok), 256-byte aligned, needs
 * no initialisation. */
size_t chimere_moe_prefill_workspace_size(const chimere_moe_layer *layer, int max_ntok);
void chimere_moe_prefill(const chimere_moe_layer *layer, const float *x, float *out, int ntok,
                         int *ids_out, float *w_out, void *workspace, size_t workspace_bytes,
                         hipStream_t stream);

/* Expert FFN on unquantized activations, IQ3_S experts: replaces the
 * reference's fused_moe_iq3s (cs/src/kernels/fused_moe.rs:345-468, kernel
 * :261-311 = cs/kernels/chimere_kernels.cu:1093-1143), its GPU path when the
 * ggml Q8_1 kernels are not selected (cs/src/qwen35_model/moe_ffn.rs:1476-1500).
 * For k < top_k, e = expert_ids[k] (device array; each id must index an expert
 * of the stacked tensors): g = G_e x, u = U_e x with f32 x = hidden,
 * h = silu(g) * u, y_k = D_e h, and output[r] += sum_k expert_weights[k] * y_k[r]
 * (output accumulates, as the reference's atomicAdd does: zero it first for
 * the bare FFN).  gate_exps / up_exps hold [E][expert_ffn rows][hidden_size]
 * IQ3_S, down_exps [E][hidden_size rows][expert_ffn], expert_bytes_* apart.
 * Unlike the reference (atomicAdd in block order), the sum over k is in
 * ascending k and every dot has a fixed order, so results repeat bit for bit.
 * hidden_size a multiple of 256 up to 4096, expert_ffn a multiple of 256 up to
 * 512, top_k 1..16; weights 4-byte aligned, hidden 16-byte aligned.  The
 * workspace (h of every expert) is chimere_fused_moe_iq3s_workspace_size
 * bytes, 16-byte aligned; no allocation. */
size_t chimere_fused_moe_iq3s_workspace_size(int hidden_size, int expert_ffn, int top_k);
void chimere_fused_moe_iq3s(const float *hidden, const void *gate_exps, const void *up_exps,
                            const void *down_exps, const int *expert_ids, const float *expert_weights,
                            float *output, int hidden_size, int expert_ffn, int64_t expert_bytes_gate,
                            int64_t expert_bytes_up, int64_t expert_bytes_down, int top_k,
                            void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ----------------------------------------------- weight quantizers (GPU) */
/* Not part of the reference's ABI (its weights come pre-quantized from GGUF);
 * used to build synthetic weights on the device.  n multiple of 32 (IQ3_S:
 * 256).  Q8_0: src/kernels/kv_q8_0.rs:49-89; Q4_0: ggml reference rule;
 * IQ3_S: this library's encoder (nearest codebook point per 4 values). */
void chimere_quantize_weights(int type, const float *x, void *out, int64_t n,
                              hipStream_t stream);

/* ------------------------------------------------------------ debug */
/* Exact int32 per-block dots: out[r*(ncols/32) + b] (IQ3_S: per 32-element
 * sub-block, already multiplied by its (1 + 2*scale); Q4_K / Q5_K: sc*sum q*q_x
 * without the min term; Q6_K: sc_lo*sum_lo + sc_hi*sum_hi of q-32).  type is a
 * ggml id: Q4_0 2, Q8_0 8, Q4_K 12, Q5_K 13, Q6_K 14, IQ3_S 21, MXFP4 39. */
void chimere_dbg_block_dots(int type, const void *weights, const void *input_q8,
                            int32_t *out, int ncols, int nrows, hipStream_t stream);

/* ------------------------------------------------------------ errors */
/* Last error on the calling host thread (CHIMERE_OK if none); clears it. */
int chimere_hip_get_last_error(void);
const char *chimere_hip_get_last_error_string(void);

#ifdef __cplusplus
}
#endif
#endif
