// ggml_gpu.cpp -- C++ host layer over libchimere_hip.so / libchimere_cpu.so
// (the counterpart of chimere-server/src/kernels/ggml_gpu.rs and of the
// layer sequences of chimere-server/src/qwen35_model/moe_ffn.rs).
#include "ggml_gpu.hpp"

#include <new>

#include "chimere_cpu.h"

namespace chimere {
namespace host {

namespace {
constexpr int T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ3_S = 21, T_MXFP4 = 39;

int nrows_y(int ncols) { return (int)(pad((size_t)ncols, MATRIX_ROW_PADDING) / Q8_1_BLOCK_ELEMS); }

}  // namespace

void check() {
    const char* msg = chimere_hip_get_last_error_string();
    const std::string m = msg ? msg : "";
    const int code = chimere_hip_get_last_error();
    if (code != CHIMERE_OK) throw Error(code, "chimere_hip error " + std::to_string(code) + ": " + m);
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(CHIMERE_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
}

GgmlGpuBuffers GgmlGpuBuffers::with_moe(size_t max_ncols, size_t max_nrows, size_t expert_ffn, size_t hidden_size,
                                        size_t top_k) {
    GgmlGpuBuffers b;
    b.max_ncols_padded = pad(max_ncols, MATRIX_ROW_PADDING);
    const size_t q8 = b.max_ncols_padded / Q8_1_BLOCK_ELEMS * Q8_1_BLOCK_BYTES;
    const size_t k = top_k ? top_k : 1, f = expert_ffn ? expert_ffn : 1, h = hidden_size ? hidden_size : 1;
    b.q8_input = DeviceBuffer<uint8_t>(q8);
    b.q8_input_b = DeviceBuffer<uint8_t>(q8);
    b.output = DeviceBuffer<float>(max_nrows ? max_nrows : 1);
    b.batched_gate = DeviceBuffer<float>(k * f);
    b.batched_up = DeviceBuffer<float>(k * f);
    b.batched_down = DeviceBuffer<float>(k * h);
    b.batched_q8_inter = DeviceBuffer<uint8_t>(k * q8_1_row_bytes((int)f));
    // the Rust buffers are zero-initialised (alloc_zeros)
    hip_check(hipMemset(b.q8_input.get(), 0, q8), "hipMemset");
    hip_check(hipMemset(b.q8_input_b.get(), 0, q8), "hipMemset");
    hip_check(hipMemset(b.batched_q8_inter.get(), 0, b.batched_q8_inter.size()), "hipMemset");
    return b;
}

// ------------------------------------------------------------ quantize
void ggml_gpu_quantize_q8_1(const float* input, void* q8_output, int ncols, hipStream_t s) {
    chimere_quantize_q8_1(input, q8_output, ncols, (int64_t)pad((size_t)ncols, MATRIX_ROW_PADDING), s);
    check();
}
void ggml_gpu_quantize_q8_1_batched(const float* input, void* q8_output, int ncols, int batch, hipStream_t s) {
    chimere_quantize_q8_1_batched(input, q8_output, ncols, (int64_t)pad((size_t)ncols, MATRIX_ROW_PADDING), batch,
                                  s);
    check();
}

// ---------------------------------------------------------------- GEMV
#define CHIMERE_GEMV_Q8(NAME, FN)                                                                            \
    void NAME(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s) {       \
        FN(w, q8_input, out, ncols, nrows, nrows_y(ncols), s);                                               \
        check();                                                                                             \
    }
CHIMERE_GEMV_Q8(ggml_gpu_gemv_iq3s_q8, chimere_mmvq_iq3s)
CHIMERE_GEMV_Q8(ggml_gpu_gemv_q8_0_q8, chimere_mmvq_q8_0)
CHIMERE_GEMV_Q8(ggml_gpu_gemv_q4_0_q8, chimere_mmvq_q4_0)
CHIMERE_GEMV_Q8(ggml_gpu_gemv_q5k_q8, chimere_mmvq_q5k)
CHIMERE_GEMV_Q8(ggml_gpu_gemv_q4k_q8, chimere_mmvq_q4k)
CHIMERE_GEMV_Q8(ggml_gpu_gemv_q6k_q8, chimere_mmvq_q6k)
CHIMERE_GEMV_Q8(ggml_gpu_gemv_mxfp4_q8, chimere_mmvq_mxfp4)
#undef CHIMERE_GEMV_Q8

#define CHIMERE_GEMV_F32(NAME, FN)                                                                           \
    void NAME(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,            \
              hipStream_t s) {                                                                               \
        FN(w, in, out, ncols, nrows, (int)pad((size_t)ncols, MATRIX_ROW_PADDING), q8_scratch, s);             \
        check();                                                                                             \
    }
CHIMERE_GEMV_F32(ggml_gpu_gemv_iq3s_f32, chimere_mmvq_iq3s_f32)
CHIMERE_GEMV_F32(ggml_gpu_gemv_q8_0_f32, chimere_mmvq_q8_0_f32)
CHIMERE_GEMV_F32(ggml_gpu_gemv_q4_0_f32, chimere_mmvq_q4_0_f32)
CHIMERE_GEMV_F32(ggml_gpu_gemv_q5k_f32, chimere_mmvq_q5k_f32)
CHIMERE_GEMV_F32(ggml_gpu_gemv_q4k_f32, chimere_mmvq_q4k_f32)
CHIMERE_GEMV_F32(ggml_gpu_gemv_q6k_f32, chimere_mmvq_q6k_f32)
#undef CHIMERE_GEMV_F32

void ggml_gpu_gemv_mxfp4_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                             hipStream_t s) {
    // the reference's argument order for this one: scratch before output (ggml_cuda_gemv.cu:448)
    chimere_mmvq_mxfp4_f32(w, in, q8_scratch, out, ncols, nrows, (int)pad((size_t)ncols, MATRIX_ROW_PADDING), s);
    check();
}

#define CHIMERE_GEMV_BATCHED(NAME, FN)                                                                       \
    void NAME(const void* all_w, const void* q8_input, float* out, const int* expert_ids, int nrows,         \
              int ncols, int64_t expert_stride, int64_t input_stride, int top_k, hipStream_t s) {            \
        FN(all_w, q8_input, out, expert_ids, ncols, nrows, nrows_y(ncols), expert_stride, input_stride,      \
           top_k, s);                                                                                        \
        check();                                                                                             \
    }
CHIMERE_GEMV_BATCHED(ggml_gpu_gemv_iq3s_batched, chimere_mmvq_iq3s_batched)
CHIMERE_GEMV_BATCHED(ggml_gpu_gemv_q8_0_batched, chimere_mmvq_q8_0_batched)
CHIMERE_GEMV_BATCHED(ggml_gpu_gemv_q4_0_batched, chimere_mmvq_q4_0_batched)
CHIMERE_GEMV_BATCHED(ggml_gpu_gemv_mxfp4_batched, chimere_mmvq_mxfp4_batched)
#undef CHIMERE_GEMV_BATCHED

void gemv_q8(int type, const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s) {
    switch (type) {
    case T_IQ3_S: return ggml_gpu_gemv_iq3s_q8(w, q8_input, out, nrows, ncols, s);
    case T_Q8_0: return ggml_gpu_gemv_q8_0_q8(w, q8_input, out, nrows, ncols, s);
    case T_Q4_0: return ggml_gpu_gemv_q4_0_q8(w, q8_input, out, nrows, ncols, s);
    case T_Q5_K: return ggml_gpu_gemv_q5k_q8(w, q8_input, out, nrows, ncols, s);
    case T_Q4_K: return ggml_gpu_gemv_q4k_q8(w, q8_input, out, nrows, ncols, s);
    case T_Q6_K: return ggml_gpu_gemv_q6k_q8(w, q8_input, out, nrows, ncols, s);
    case T_MXFP4: return ggml_gpu_gemv_mxfp4_q8(w, q8_input, out, nrows, ncols, s);
    default: throw Error(CHIMERE_ERR_ARG, "gemv_q8: unsupported type " + std::to_string(type));
    }
}

void gemv_f32(int type, const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
              hipStream_t s) {
    switch (type) {
    case T_IQ3_S: return ggml_gpu_gemv_iq3s_f32(w, in, out, q8_scratch, nrows, ncols, s);
    case T_Q8_0: return ggml_gpu_gemv_q8_0_f32(w, in, out, q8_scratch, nrows, ncols, s);
    case T_Q4_0: return ggml_gpu_gemv_q4_0_f32(w, in, out, q8_scratch, nrows, ncols, s);
    case T_Q5_K: return ggml_gpu_gemv_q5k_f32(w, in, out, q8_scratch, nrows, ncols, s);
    case T_Q4_K: return ggml_gpu_gemv_q4k_f32(w, in, out, q8_scratch, nrows, ncols, s);
    case T_Q6_K: return ggml_gpu_gemv_q6k_f32(w, in, out, q8_scratch, nrows, ncols, s);
    case T_MXFP4: return ggml_gpu_gemv_mxfp4_f32(w, in, out, q8_scratch, nrows, ncols, s);
    default: throw Error(CHIMERE_ERR_ARG, "gemv_f32: unsupported type " + std::to_string(type));
    }
}

void gemv_batched(int type, const void* all_w, const void* q8_input, float* out, const int* expert_ids, int nrows,
                  int ncols, int64_t expert_stride, int64_t input_stride, int top_k, hipStream_t s) {
    switch (type) {
    case T_IQ3_S:
        return ggml_gpu_gemv_iq3s_batched(all_w, q8_input, out, expert_ids, nrows, ncols, expert_stride, input_stride,
                                          top_k, s);
    case T_Q8_0:
        return ggml_gpu_gemv_q8_0_batched(all_w, q8_input, out, expert_ids, nrows, ncols, expert_stride, input_stride,
                                          top_k, s);
    case T_Q4_0:
        return ggml_gpu_gemv_q4_0_batched(all_w, q8_input, out, expert_ids, nrows, ncols, expert_stride, input_stride,
                                          top_k, s);
    case T_MXFP4:
        return ggml_gpu_gemv_mxfp4_batched(all_w, q8_input, out, expert_ids, nrows, ncols, expert_stride,
                                           input_stride, top_k, s);
    default: throw Error(CHIMERE_ERR_ARG, "gemv_batched: unsupported type " + std::to_string(type));
    }
}

// ------------------------------------------------------ routing / glue
void raw_f32_gemv(const float* A, const float* x, float* y, int rows, int cols, hipStream_t s) {
    chimere_f32_gemv(A, x, y, rows, cols, s);
    check();
}
void gpu_topk_softmax(const float* logits, int* top_idx, float* top_w, int num_experts, int top_k, int ntok,
                      hipStream_t s) {
    chimere_topk_softmax(logits, top_idx, top_w, num_experts, top_k, ntok, s);
    check();
}
void silu_mul_inplace(float* gate, const float* up, int n, hipStream_t s) {
    chimere_silu_mul_inplace(gate, up, n, s);
    check();
}
void weighted_combine_gpu(const float* expert_outputs, const float* weights, float* accum, int hidden_size,
                          int top_k, hipStream_t s) {
    chimere_weighted_combine(expert_outputs, weights, accum, hidden_size, top_k, s);
    check();
}
void raw_sigmoid_gate_add_inplace(float* output, const float* gate, const float* combined, int n, hipStream_t s) {
    chimere_sigmoid_gate_add(output, gate, combined, n, s);
    check();
}

// ------------------------------------------------------------ MoE layer
MoeLayer::MoeLayer(const chimere_moe_layer& c, int max_ntok, hipStream_t s) : c_(c), max_ntok_(max_ntok) {
    const size_t wb = chimere_moe_workspace_size(&c_, max_ntok);
    check();
    if (wb == 0) throw Error(CHIMERE_ERR_ARG, "chimere_moe_workspace_size rejected the layer shape");
    ws_ = DeviceBuffer<uint8_t>(wb);
    chimere_moe_workspace_init(ws_.get(), wb, s);
    check();
    const int H = c_.hidden, F = c_.ffn, E = c_.n_experts, K = c_.top_k;
    bufs_ = GgmlGpuBuffers::with_moe((size_t)(H > F ? H : F), (size_t)(H > F ? H : F), (size_t)F, (size_t)H,
                                     (size_t)K);
    pair_ = DeviceBuffer<float>(2 * (size_t)(E > H ? E : H));
    one_ = DeviceBuffer<float>(4);
    const float ones[4] = {1.0f, 1.0f, 1e30f, 0.0f};   // two unit weights; a gate logit with sigmoid == 1
    hip_check(hipMemcpy(one_.get(), ones, sizeof(ones), hipMemcpyHostToDevice), "hipMemcpy");
    if (c_.logit_bias)   // row 1 of pair_: the bias, added to row 0's logits by a two-row combine
        hip_check(hipMemcpy(pair_.get() + E, c_.logit_bias, sizeof(float) * E, hipMemcpyDeviceToDevice), "hipMemcpy");
    shg_ = DeviceBuffer<float>((size_t)F);
    shu_ = DeviceBuffer<float>((size_t)F);
    shd_ = DeviceBuffer<float>((size_t)H);
    glogit_ = DeviceBuffer<float>(1);
    accum_ = DeviceBuffer<float>((size_t)H);
    sel_ = DeviceBuffer<float>((size_t)E);
}

void MoeLayer::forward(const float* x, float* out, int ntok, int* ids, float* w, hipStream_t s) {
    if (ntok < 1 || ntok > max_ntok_) throw Error(CHIMERE_ERR_ARG, "forward: ntok out of range");
    chimere_moe_ffn_decode(&c_, x, out, ntok, ids, w, ws_.get(), ws_.size(), s);
    check();
}

// router GEMV (+ bias) and top-k softmax (moe_ffn.rs:1094-1140)
void MoeLayer::route(const float* x, int* ids, float* w, hipStream_t s) {
    const int E = c_.n_experts;
    float* logits = pair_.get();
    raw_f32_gemv(c_.router_w, x, logits, E, c_.hidden, s);
    const float* sel = logits;
    if (c_.logit_bias) {
        // logits + bias: fmaf(1, bias, fmaf(1, logits, 0)) = logits + bias
        weighted_combine_gpu(pair_.get(), one_.get(), sel_.get(), E, 2, s);
        sel = sel_.get();
    }
    gpu_topk_softmax(sel, ids, w, E, c_.top_k, 1, s);
}

// shared expert and the final combine (moe_ffn.rs:1597-1761):
// out = shared * sigmoid(<x, gate_w>) + accum (ungated: shared + accum)
void MoeLayer::shared_tail(const float* x, const float* accum, float* out, hipStream_t s) {
    const int H = c_.hidden, F = c_.ffn, st = c_.shared_type;
    if (st < 0) {
        hip_check(hipMemcpyAsync(out, accum, sizeof(float) * H, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
        return;
    }
    gemv_f32(st, c_.sh_gate, x, shg_.get(), bufs_.q8_input.get(), F, H, s);
    gemv_q8(st, c_.sh_up, bufs_.q8_input.get(), shu_.get(), F, H, s);
    silu_mul_inplace(shg_.get(), shu_.get(), F, s);
    gemv_f32(st, c_.sh_down, shg_.get(), shd_.get(), bufs_.q8_input_b.get(), H, F, s);
    const float* gate = one_.get() + 2;
    if (c_.sh_gate_w) {
        raw_f32_gemv(c_.sh_gate_w, x, glogit_.get(), 1, H, s);
        gate = glogit_.get();
    }
    raw_sigmoid_gate_add_inplace(shd_.get(), gate, accum, H, s);
    hip_check(hipMemcpyAsync(out, shd_.get(), sizeof(float) * H, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
}

void MoeLayer::forward_v3(const float* x, float* out, int* ids, float* w, hipStream_t s) {
    const int H = c_.hidden, F = c_.ffn, K = c_.top_k, t = c_.expert_type;
    route(x, ids, w, s);
    ggml_gpu_quantize_q8_1(x, bufs_.q8_input.get(), H, s);
    gemv_batched(t, c_.gate_exps, bufs_.q8_input.get(), bufs_.batched_gate.get(), ids, F, H, c_.gate_stride, 0, K, s);
    gemv_batched(t, c_.up_exps, bufs_.q8_input.get(), bufs_.batched_up.get(), ids, F, H, c_.up_stride, 0, K, s);
    silu_mul_inplace(bufs_.batched_gate.get(), bufs_.batched_up.get(), K * F, s);
    ggml_gpu_quantize_q8_1_batched(bufs_.batched_gate.get(), bufs_.batched_q8_inter.get(), F, K, s);
    gemv_batched(t, c_.down_exps, bufs_.batched_q8_inter.get(), bufs_.batched_down.get(), ids, H, F, c_.down_stride,
                 (int64_t)q8_1_row_bytes(F), K, s);
    weighted_combine_gpu(bufs_.batched_down.get(), w, accum_.get(), H, K, s);
    shared_tail(x, accum_.get(), out, s);
}

void MoeLayer::attach_cpu_experts(const uint8_t* gate, const uint8_t* up, const uint8_t* down) {
    if (c_.expert_type != T_IQ3_S) throw Error(CHIMERE_ERR_ARG, "the host expert path takes IQ3_S experts only");
    cg_ = gate;
    cu_ = up;
    cd_ = down;
    h_x_.resize((size_t)c_.hidden);
    h_acc_.resize((size_t)c_.hidden);
    h_ids_.resize((size_t)c_.top_k);
    h_w_.resize((size_t)c_.top_k);
}

void MoeLayer::forward_ncmoe(const float* x, float* out, int* ids, float* w, int nthreads, hipStream_t s) {
    if (!cg_) throw Error(CHIMERE_ERR_ARG, "forward_ncmoe: attach_cpu_experts() first");
    const int H = c_.hidden, F = c_.ffn, K = c_.top_k;
    route(x, ids, w, s);
    hip_check(hipMemcpyAsync(h_ids_.data(), ids, sizeof(int32_t) * K, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    hip_check(hipMemcpyAsync(h_w_.data(), w, sizeof(float) * K, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    hip_check(hipMemcpyAsync(h_x_.data(), x, sizeof(float) * H, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    const int rc = chimere_ncmoe_experts(cg_, cu_, cd_, (size_t)c_.gate_stride, (size_t)c_.up_stride,
                                         (size_t)c_.down_stride, h_ids_.data(), h_w_.data(), K, h_x_.data(),
                                         h_acc_.data(), H, F, c_.n_experts, nthreads);
    if (rc == CHIMERE_CPU_ENOMEM) throw std::bad_alloc();   // a host allocation failed, not a bad argument
    if (rc != CHIMERE_CPU_OK) throw Error(CHIMERE_ERR_ARG, "chimere_ncmoe_experts rejected its arguments");
    hip_check(hipMemcpyAsync(accum_.get(), h_acc_.data(), sizeof(float) * H, hipMemcpyHostToDevice, s),
              "hipMemcpyAsync");
    shared_tail(x, accum_.get(), out, s);
    // h_acc_ is reused by the next call: the copy must have left it
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

}  // namespace host
}  // namespace chimere
