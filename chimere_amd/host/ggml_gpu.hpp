// ggml_gpu.hpp -- C++ host layer over libchimere_hip.so / libchimere_cpu.so:
// the counterpart of the reference's Rust host code for this path.
//
//  * ggml_gpu_* free functions and GgmlGpuBuffers mirror
//    chimere-server/src/kernels/ggml_gpu.rs (buffers :292-443, wrappers
//    :445-1488): same names, argument order and meaning (nrows / ncols are a
//    GEMV's output / input sizes, strides in bytes).  Where a Rust wrapper
//    returns Result<()>, these throw chimere::host::Error when the library
//    rejected the call (chimere_hip_get_last_error).
//  * raw_f32_gemv / gpu_topk_softmax / silu_mul_inplace / weighted_combine_gpu
//    / raw_sigmoid_gate_add_inplace mirror the glue kernels' wrappers
//    (elementwise.rs:599, topk_softmax.rs:113, fused_ops.rs:34 / :364,
//    scratch_pool.rs:264).
//  * MoeLayer holds one layer (the C ABI's chimere_moe_layer plus its
//    workspace) and runs it three ways, as chimere-server's moe_ffn.rs does:
//    forward() = the fused entry point, forward_v3() = the reference's
//    7-launch V3 sequence (moe_ffn.rs:1185-1384) + shared expert
//    (:1597-1761), forward_ncmoe() = routed experts on the host cores
//    (:1507-1591) through libchimere_cpu.so.
//
// Every device pointer is caller-owned except the buffers GgmlGpuBuffers and
// MoeLayer allocate (freed by their destructors).
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "chimere_hip.h"

namespace chimere {
namespace host {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

// Throws Error if the last C-ABI call on this thread recorded an error.
void check();
// HIP runtime status -> Error
void hip_check(hipError_t e, const char* what);

constexpr int Q8_1_BLOCK_BYTES = 36, Q8_1_BLOCK_ELEMS = 32, MATRIX_ROW_PADDING = 512;
inline size_t pad(size_t n, size_t align) { return (n + align - 1) / align * align; }   // ggml_gpu.rs:55
inline size_t q8_1_row_bytes(int ncols) {
    return pad((size_t)ncols, MATRIX_ROW_PADDING) / Q8_1_BLOCK_ELEMS * Q8_1_BLOCK_BYTES;
}

// Device allocation owned by the host layer.
template <typename T>
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n) : n_(n) {
        if (n) hip_check(hipMalloc((void**)&p_, n * sizeof(T)), "hipMalloc");
    }
    ~DeviceBuffer() { if (p_) (void)hipFree(p_); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) { if (p_) (void)hipFree(p_); p_ = o.p_; n_ = o.n_; o.p_ = nullptr; o.n_ = 0; }
        return *this;
    }
    T* get() const { return p_; }
    size_t size() const { return n_; }

private:
    T* p_ = nullptr;
    size_t n_ = 0;
};

// ggml_gpu.rs:292-443: preallocated Q8_1 / batched-MoE scratch and the
// stream the wrappers launch on.
struct GgmlGpuBuffers {
    DeviceBuffer<uint8_t> q8_input, q8_input_b;
    DeviceBuffer<float> output;
    size_t max_ncols_padded = 0;
    DeviceBuffer<float> batched_gate, batched_up, batched_down;
    DeviceBuffer<uint8_t> batched_q8_inter;

    static GgmlGpuBuffers create(size_t max_ncols, size_t max_nrows) { return with_moe(max_ncols, max_nrows, 0, 0, 0); }
    static GgmlGpuBuffers with_moe(size_t max_ncols, size_t max_nrows, size_t expert_ffn, size_t hidden_size,
                                   size_t top_k);
    void set_stream_override(hipStream_t s) { stream_override_ = s; }
    void clear_stream_override() { stream_override_ = nullptr; }
    hipStream_t active_stream() const { return stream_override_; }

private:
    hipStream_t stream_override_ = nullptr;
};

// ------------------------------------------------------------ quantize
void ggml_gpu_quantize_q8_1(const float* input, void* q8_output, int ncols, hipStream_t s);
void ggml_gpu_quantize_q8_1_batched(const float* input, void* q8_output, int ncols, int batch, hipStream_t s);

// ---------------------------------------------------------------- GEMV
// pre-quantized Q8_1 input (ggml_gpu.rs:714, :747)
void ggml_gpu_gemv_iq3s_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void ggml_gpu_gemv_q8_0_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void ggml_gpu_gemv_q4_0_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void ggml_gpu_gemv_q5k_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void ggml_gpu_gemv_q4k_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void ggml_gpu_gemv_q6k_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void ggml_gpu_gemv_mxfp4_q8(const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
// fused f32 -> Q8_1 -> GEMV (ggml_gpu.rs:834-1060)
void ggml_gpu_gemv_iq3s_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                            hipStream_t s);
void ggml_gpu_gemv_q8_0_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                            hipStream_t s);
void ggml_gpu_gemv_q4_0_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                            hipStream_t s);
void ggml_gpu_gemv_q5k_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                           hipStream_t s);
void ggml_gpu_gemv_q4k_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                           hipStream_t s);
void ggml_gpu_gemv_q6k_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                           hipStream_t s);
void ggml_gpu_gemv_mxfp4_f32(const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
                             hipStream_t s);
// top_k expert GEMVs with device-resident ids (ggml_gpu.rs:1225)
void ggml_gpu_gemv_iq3s_batched(const void* all_w, const void* q8_input, float* out, const int* expert_ids,
                                int nrows, int ncols, int64_t expert_stride, int64_t input_stride, int top_k,
                                hipStream_t s);
void ggml_gpu_gemv_q8_0_batched(const void* all_w, const void* q8_input, float* out, const int* expert_ids,
                                int nrows, int ncols, int64_t expert_stride, int64_t input_stride, int top_k,
                                hipStream_t s);
void ggml_gpu_gemv_q4_0_batched(const void* all_w, const void* q8_input, float* out, const int* expert_ids,
                                int nrows, int ncols, int64_t expert_stride, int64_t input_stride, int top_k,
                                hipStream_t s);
void ggml_gpu_gemv_mxfp4_batched(const void* all_w, const void* q8_input, float* out, const int* expert_ids,
                                 int nrows, int ncols, int64_t expert_stride, int64_t input_stride, int top_k,
                                 hipStream_t s);
// type-dispatched forms used by the layer sequences
void gemv_q8(int type, const void* w, const void* q8_input, float* out, int nrows, int ncols, hipStream_t s);
void gemv_f32(int type, const void* w, const float* in, float* out, void* q8_scratch, int nrows, int ncols,
              hipStream_t s);
void gemv_batched(int type, const void* all_w, const void* q8_input, float* out, const int* expert_ids, int nrows,
                  int ncols, int64_t expert_stride, int64_t input_stride, int top_k, hipStream_t s);

// ------------------------------------------------------ routing / glue
void raw_f32_gemv(const float* A, const float* x, float* y, int rows, int cols, hipStream_t s);
void gpu_topk_softmax(const float* logits, int* top_idx, float* top_w, int num_experts, int top_k, int ntok,
                      hipStream_t s);
void silu_mul_inplace(float* gate, const float* up, int n, hipStream_t s);
void weighted_combine_gpu(const float* expert_outputs, const float* weights, float* accum, int hidden_size,
                          int top_k, hipStream_t s);
void raw_sigmoid_gate_add_inplace(float* output, const float* gate, const float* combined, int n, hipStream_t s);

// ------------------------------------------------------------ MoE layer
class MoeLayer {
public:
    // `c` describes device tensors the caller keeps alive; max_ntok <= 8.
    MoeLayer(const chimere_moe_layer& c, int max_ntok = 8, hipStream_t s = nullptr);
    const chimere_moe_layer& desc() const { return c_; }

    // x [ntok, H] -> out [ntok, H] through chimere_moe_ffn_decode; ids / w
    // [ntok, K] receive the routing when non-null.
    void forward(const float* x, float* out, int ntok, int* ids, float* w, hipStream_t s);
    // One token through the reference's V3 launch sequence and shared expert.
    void forward_v3(const float* x, float* out, int* ids, float* w, hipStream_t s);
    // One token with the routed experts on the host (IQ3_S experts): host
    // copies [E * expert_bytes] of gate / up / down, nthreads host threads.
    void attach_cpu_experts(const uint8_t* gate, const uint8_t* up, const uint8_t* down);
    // Throws Error(CHIMERE_ERR_ARG) for rejected arguments, std::bad_alloc
    // when the host expert loop cannot allocate.
    void forward_ncmoe(const float* x, float* out, int* ids, float* w, int nthreads, hipStream_t s);

private:
    void route(const float* x, int* ids, float* w, hipStream_t s);
    void shared_tail(const float* x, const float* accum, float* out, hipStream_t s);

    chimere_moe_layer c_;
    int max_ntok_;
    DeviceBuffer<uint8_t> ws_;
    GgmlGpuBuffers bufs_;
    DeviceBuffer<float> pair_;    // router logits and bias rows / two addends
    DeviceBuffer<float> one_;     // gate logit whose sigmoid is exactly 1
    DeviceBuffer<float> shg_, shu_, shd_, glogit_, accum_, sel_;
    const uint8_t *cg_ = nullptr, *cu_ = nullptr, *cd_ = nullptr;
    std::vector<float> h_x_, h_w_, h_acc_;
    std::vector<int32_t> h_ids_;
};

}  // namespace host
}  // namespace chimere
