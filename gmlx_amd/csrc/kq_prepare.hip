// bf16 / fp32 activations into the fp16 rows every matmul and gather kernel
// reads, without losing range:
//
//   x16[r][k] = fp16(x[r][k] * 2^-e[r]),   e[r] = E - 15 where max_k |x[r][k]| = f 2^E, f in [0.5, 1)
//
// so each row's largest magnitude lands in [2^14, 2^15) (below fp16's 65504)
// and the kernels multiply their fp32 results by 2^e[r] before any bias or
// activation (ldexp: exact).  A bf16 value keeps all its bits (8-bit mantissa
// inside fp16's 11) unless it lies more than 2^29 below its row's maximum,
// where fp16 turns subnormal; such entries add at most 2^-29 of the largest
// term each.  An fp32 value rounds once to 11 bits, as before, but no longer
// overflows past 65504 or flushes below 2^-14.  Rows of zeros get e = 0; inf
// and NaN pass through (e = 0 for a row whose maximum is not finite).
//
// This replaces the reference's convert-on-load of bf16 / fp32 operands
// (accumulate in fp32, gmlx/dtypes.py:8-9, 16-17, 26-29): the MFMA path of
// these kernels takes fp16 operands, and the per-row power of two keeps the
// conversion exact for bf16.
#include "kq_common.h"

namespace {

template <int XT>
__device__ __forceinline__ float load_elem(const char *row, int k) {
    if constexpr (XT == 2) return ((const float *)row)[k];
    else return kq_bf16_bits_to_f32(((const uint16_t *)row)[k]);
}

// One workgroup per row: the row's maximum magnitude, then the scaled fp16 row.
template <int XT>
__global__ __launch_bounds__(256) void prepare_rows_kernel(const char *x, int64_t stride_bytes, int K,
                                                           kq_half *x16, int32_t *e_out) {
    __shared__ float part[4];
    const int r = (int)blockIdx.x;
    const char *row = x + (int64_t)r * stride_bytes;
    float mx = 0.f;
    for (int k = (int)threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(load_elem<XT>(row, k)));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    int e = 0;
    if (mx > 0.f && mx <= 3.402823466e38f) {
        int E;
        (void)frexpf(mx, &E);
        e = E - 15;
    }
    if (threadIdx.x == 0) e_out[r] = e;
    kq_half *dst = x16 + (int64_t)r * K;
    for (int k = (int)threadIdx.x; k < K; k += 256) dst[k] = (kq_half)ldexpf(load_elem<XT>(row, k), -e);
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

size_t kq_prepared_bytes(int64_t rows, int64_t K) {
    return align256((size_t)rows * (size_t)K * 2) + align256((size_t)rows * 4);
}

// rows x K activations of x_dtype (bf16 or fp32), x_stride elements apart ->
// fp16 rows (K apart) at `out` and their exponents right after
// (kq_prepared_bytes(rows, K) bytes, 256-aligned parts).
int kq_prepare_rows(const void *x, int x_dtype, int64_t x_stride, int32_t rows, int32_t K, void *out,
                    const int32_t **exp_out, const void **x16_out, hipStream_t s) {
    kq_half *x16 = (kq_half *)out;
    int32_t *e = (int32_t *)((char *)out + align256((size_t)rows * (size_t)K * 2));
    *x16_out = x16;
    *exp_out = e;
    if (rows <= 0) return KQ_OK;
    if (x_dtype == KQ_DTYPE_F32)
        hipLaunchKernelGGL(prepare_rows_kernel<2>, dim3(rows), dim3(256), 0, s, (const char *)x, x_stride * 4, K,
                           x16, e);
    else
        hipLaunchKernelGGL(prepare_rows_kernel<1>, dim3(rows), dim3(256), 0, s, (const char *)x, x_stride * 2, K,
                           x16, e);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}
