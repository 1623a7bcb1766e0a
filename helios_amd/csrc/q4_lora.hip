// LoRA delta on a quantized projection's output (native_model.cc:316-328):
//   y = model_dtype(base + model_dtype((float32(x) . A^T) . B^T * scale))
// A [rank, K] and B [N, rank] are fp32 (the adapter's tensors cast to float32,
// native_model.cc:3420-3426).  Two small passes after the base qmm, which has
// already written base (bf16 in the bf16 model dtype, else fp32) into y:
//   lora_down: t[m, r] = sum_k x[m, k] A[r, k]            (fp32, one wave per (m, r))
//   lora_up:   y[m, n] = y[m, n] + delta,  delta = (sum_r t[m, r] B[n, r]) * scale
// In bf16 the scale is bf16 (model_scalar) and delta is rounded to bf16 before the
// bf16 add, as the reference's array ops round.
#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

__global__ __launch_bounds__(256) void lora_down_kernel(const uint16_t* __restrict__ x, const float* __restrict__ a,
                                                        float* __restrict__ t, int m_rows, int rank, int k) {
    const int wave = (int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    if (wave >= m_rows * rank) return;  // whole waves leave together
    const int m = wave / rank, r = wave - m * rank;
    const uint16_t* xr = x + (long)m * k;
    const float* ar = a + (long)r * k;
    float acc = 0.f;
    for (int c = lane; c < k; c += 64) acc = __builtin_fmaf(bf16_lo((uint32_t)xr[c]), ar[c], acc);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d);
    if (lane == 0) t[(long)m * rank + r] = acc;
}

template <bool F32>
__global__ __launch_bounds__(256) void lora_up_kernel(const float* __restrict__ t, const float* __restrict__ b,
                                                      void* __restrict__ y, int m_rows, int n_rows, int rank,
                                                      float scale) {
#pragma clang fp contract(off)
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)m_rows * n_rows) return;
    const int m = (int)(i / n_rows);
    const int n = (int)(i - (long)m * n_rows);
    const float* tr = t + (long)m * rank;
    const float* br = b + (long)n * rank;
    float d = 0.f;
    for (int r = 0; r < rank; ++r) d = __builtin_fmaf(tr[r], br[r], d);
    if (F32) {
        float* yf = static_cast<float*>(y);
        yf[i] = yf[i] + d * scale;
    } else {
        uint16_t* yb = static_cast<uint16_t*>(y);
        const float base = __uint_as_float((uint32_t)yb[i] << 16);
        yb[i] = f32_to_bf16(base + round_bf16(d * round_bf16(scale)));
    }
}

}  // namespace

hipError_t launch_lora(const uint16_t* x, const float* a, const float* b, float* t, void* y, int m, int n, int k,
                       int rank, float scale, bool out_f32, hipStream_t stream) {
    const long waves = (long)m * rank;
    hipLaunchKernelGGL(lora_down_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, x, a, t, m, rank, k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const long total = (long)m * n;
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (out_f32)
        hipLaunchKernelGGL((lora_up_kernel<true>), dim3(grid), dim3(256), 0, stream, t, b, y, m, n, rank, scale);
    else
        hipLaunchKernelGGL((lora_up_kernel<false>), dim3(grid), dim3(256), 0, stream, t, b, y, m, n, rank, scale);
    return hipGetLastError();
}

}  // namespace q4
