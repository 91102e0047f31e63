/*
 * chimere_cpu.h -- C ABI of libchimere_cpu.so, the host-side expert path
 * ("ncmoe": routed experts whose IQ3_S weights stay in host memory and are
 * evaluated on the CPU for one decode token).
 *
 * Drop-in for the reference's ggml wrapper
 *   chimere-server/ffi/ggml_iq3s_gemv.h:19-64 (implementation
 *   chimere-server/ffi/ggml_iq3s_gemv.c:33-127),
 * bound on the Rust side in chimere-server/ffi/src/lib.rs:650-681 (safe wrappers
 *   lib.rs:710-777).
 * The six ggml_ffi_* entry points keep the reference's names, signatures and
 * meaning.  chimere_ncmoe_experts() has no single counterpart: it is the
 * per-token expert loop of chimere-server/src/qwen35_model/moe_ffn.rs:1507-1591
 * (gate/up GEMV, SwiGLU, down GEMV, weighted accumulate) in one call.
 *
 * Every pointer is a HOST pointer.  Formats: IQ3_S 110 B per 256 weights;
 * Q8_K 296 B per 256 values ([f32 d][f32 sum][i8 q[256]][i16 bsums[16]]).
 * ncols / hidden_size / expert_ffn must be multiples of 256.
 */
#ifndef CHIMERE_CPU_H
#define CHIMERE_CPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHIMERE_CPU_OK 0
#define CHIMERE_CPU_EINVAL 1   /* rejected argument (null, shape, expert id, byte sizes) */
#define CHIMERE_CPU_ENOMEM 2   /* host allocation failed */

/* f32[k] -> Q8_K[k / 256]  (ggml_iq3s_gemv.h:19) */
void ggml_ffi_quantize_q8_K(const float* x, void* y, int64_t k);

/* *s = IQ3_S row (n weights) . Q8_K vector (n values)  (ggml_iq3s_gemv.h:30) */
/* The Q8_K quants are expected in [-127, 127] (the library's quantizer
 * never emits -128).  A caller-supplied -128 under a negative IQ3_S sign is
 * negated by byte wrap-around (it stays -128) on every instruction-set path,
 * as ggml's AVX2 sign instruction does. */
void ggml_ffi_vec_dot_iq3s_q8K(int n, float* s, const void* vx, const void* vy);

/* y[nrows] = W[nrows, ncols] (IQ3_S) x[ncols] (f32, quantized to Q8_K
 * inside), one thread  (ggml_iq3s_gemv.h:43) */
void ggml_ffi_gemv_iq3s(const void* w_iq3s, const float* x_f32, float* y_f32, int nrows, int ncols);

/* the same over nthreads OpenMP threads (0 = OpenMP's default); results do
 * not depend on nthreads  (ggml_iq3s_gemv.h:54) */
void ggml_ffi_gemv_iq3s_parallel(const void* w_iq3s, const float* x_f32, float* y_f32, int nrows, int ncols,
                                 int nthreads);

size_t ggml_ffi_iq3s_row_bytes(int ncols);   /* ggml_iq3s_gemv.h:60 */
size_t ggml_ffi_q8k_row_bytes(int ncols);    /* ggml_iq3s_gemv.h:64 */

/* combined[hidden_size] = sum over k of weights[k] * down_e(silu(gate_e h) * up_e h),
 * e = ids[k], in the order of ids (moe_ffn.rs:1538-1585).  The expert tensors
 * are [n_experts] consecutive slices of expert_bytes_* bytes: gate/up
 * [expert_ffn, hidden_size], down [hidden_size, expert_ffn], IQ3_S.
 * Returns CHIMERE_CPU_OK, or CHIMERE_CPU_EINVAL / _ENOMEM with combined
 * untouched.  top_k <= 64. */
int chimere_ncmoe_experts(const void* gate_exps, const void* up_exps, const void* down_exps, size_t expert_bytes_gate,
                          size_t expert_bytes_up, size_t expert_bytes_down, const int32_t* ids, const float* weights,
                          int top_k, const float* hidden, float* combined, int hidden_size, int expert_ffn,
                          int n_experts, int nthreads);

/* integer kernel in use: 2 AVX-512, 1 AVX2, 0 portable (all give the same results) */
int chimere_cpu_isa(void);

#ifdef __cplusplus
}
#endif
#endif
