// probe.hip -- attainable-rate microbenchmarks that the benchmark reports
// beside the datasheet peaks: a streaming HBM read and a dense int8 MFMA
// loop.  Built as its own library (libchimere_probe.so) that only the
// benchmark loads; the product library exports no measurement kernels.
// Entry points return 0 on success, -1 on bad arguments, -2 on a failed launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace chimere {

typedef int v4i_p __attribute__((ext_vector_type(4)));
typedef int v16i_p __attribute__((ext_vector_type(16)));

// Every thread reads 16-byte pieces grid-strided (four independent loads in
// flight per iteration, non-temporal) and folds them with xor; one word per
// work-group is written so the loads cannot be dropped.
__global__ __launch_bounds__(256) void k_stream_read(const v4i_p* __restrict__ p, int64_t n16,
                                                     uint32_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        v4i_p v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = __builtin_nontemporal_load(p + i + k * stride);
#pragma unroll
        for (int k = 0; k < 4; k++) acc ^= (uint32_t)(v[k].x ^ v[k].y ^ v[k].z ^ v[k].w);
    }
    for (; i < n16; i += stride) {
        const v4i_p v = p[i];
        acc ^= (uint32_t)(v.x ^ v.y ^ v.z ^ v.w);
    }
    __shared__ uint32_t red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0;
        for (int k = 0; k < 256; k++) r ^= red[k];
        out[blockIdx.x] = r;
    }
}

// Each wave runs 4 independent chains of iters v_mfma_i32_32x32x32_i8
// (32*32*32 multiply-adds each) on register operands.
__global__ __launch_bounds__(256) void k_mfma_i8(int iters, int32_t* __restrict__ out) {
    const int l = threadIdx.x;
    v4i_p a = {l, l * 3, l * 5, l * 7}, b = {l * 11, l * 13, 1, 2};
    v16i_p c0 = {0}, c1 = {0}, c2 = {0}, c3 = {0};
    for (int it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) s += c0[k] ^ c1[k] ^ c2[k] ^ c3[k];
    out[(int64_t)blockIdx.x * 256 + l] = s;
}

}  // namespace chimere

using namespace chimere;

extern "C" {

// nblocks work-groups of 256 threads read `bytes` (16-byte aligned) once;
// out[nblocks] receives an xor fold.
int chimere_probe_stream_read(const void* buf, int64_t bytes, uint32_t* out, int nblocks, hipStream_t s) {
    if (!buf || !out || bytes < 16 || (bytes & 15) || ((uintptr_t)buf & 15) || nblocks <= 0) return -1;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)nblocks), dim3(256), 0, s, (const v4i_p*)buf, bytes / 16, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// nblocks x 4 waves, each 4 x iters v_mfma_i32_32x32x32_i8 (65536 int8 ops
// each); out[nblocks * 256].
int chimere_probe_mfma_i8(int32_t* out, int iters, int nblocks, hipStream_t s) {
    if (!out || iters <= 0 || nblocks <= 0) return -1;
    hipLaunchKernelGGL(k_mfma_i8, dim3((unsigned)nblocks), dim3(256), 0, s, iters, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
