// LoRA delta on a quantized projection's output (native_model.cc:316-328):
//   y = model_dtype(base + model_dtype((float32(x) . A^T) . B^T * scale))
// A [rank, K] and B [N, rank] are fp32 (the adapter's tensors cast to float32,
// native_model.cc:3420-3426).  Two passes after the base qmm, which has already
// written base (bf16 in the bf16 model dtype, else fp32) into y:
//   lora_down: t[m, r] = sum_k x[m, k] A[r, k]     (fp32)
//   lora_up:   y[m, n] = y[m, n] + delta,  delta = (sum_r t[m, r] B[n, r]) * scale
// In bf16 the scale is bf16 (model_scalar) and delta is rounded to bf16 before the
// bf16 add, as the reference's array ops round.
//
// lora_down: K is cut into kSlices slices; a 256-thread workgroup per (4 rows of x,
// 16 ranks, slice) has wave w take ranks 4w..4w+3 and lane l an 8-column chunk of the
// slice per step (one 16-byte x load per row, two 16-byte A loads per rank, all in
// flight together), then each wave sums its 4 x 4 partials by shuffles and writes
// them to part[slice][m][r].  No atomics: lora_up adds the slices in a fixed order.
// lora_up: a 256-thread workgroup per (256 columns, 16 or 64 rows); t[m, r] (the
// slices summed in order) and the workgroup's rows of B are staged in LDS 16 ranks at
// a time (B with coalesced loads), each thread takes its column's B values into
// registers and updates its rows of y.  B is read once per 16 or 64 rows, y once.
#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

constexpr int kDownRows = 4;    // rows of x per lora_down workgroup
constexpr int kWaveRanks = 4;   // ranks per lora_down wave
constexpr int kRankBlock = 16;  // ranks per lora_down workgroup / per lora_up register block
constexpr int kUpRows = 16;     // rows of y per lora_up workgroup (M <= 16)
constexpr int kUpRowsLarge = 32;  // rows of y per lora_up workgroup (M > 16)

__global__ __launch_bounds__(256) void lora_down_kernel(const uint16_t* __restrict__ x, const float* __restrict__ a,
                                                        float* __restrict__ part, int m_rows, int rank, int k,
                                                        int slice_chunks) {
    const int m0 = (int)blockIdx.x * kDownRows;
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int r0 = (int)blockIdx.y * kRankBlock + wave * kWaveRanks;
    const int slice = (int)blockIdx.z;
    const int chunks = k >> 3;  // 8-column chunks (K is a multiple of 64)
    const int c_end = (slice + 1) * slice_chunks < chunks ? (slice + 1) * slice_chunks : chunks;
    float acc[kDownRows][kWaveRanks];
#pragma unroll
    for (int i = 0; i < kDownRows; ++i)
#pragma unroll
        for (int r = 0; r < kWaveRanks; ++r) acc[i][r] = 0.f;
    for (int c = slice * slice_chunks + lane; c < c_end; c += 64) {
        uint4 xu[kDownRows];
        float4 av[kWaveRanks][2];
#pragma unroll
        for (int i = 0; i < kDownRows; ++i) {
            const int m = m0 + i < m_rows ? m0 + i : m_rows - 1;  // rows past M: any row, never stored
            xu[i] = *reinterpret_cast<const uint4*>(x + (long)m * k + 8 * c);
        }
#pragma unroll
        for (int r = 0; r < kWaveRanks; ++r) {
            const int rr = r0 + r < rank ? r0 + r : rank - 1;  // ranks past the adapter's: never stored
            const float4* ap = reinterpret_cast<const float4*>(a + (long)rr * k + 8 * c);
            av[r][0] = ap[0];
            av[r][1] = ap[1];
        }
#pragma unroll
        for (int i = 0; i < kDownRows; ++i) {
            const uint32_t w[4] = {xu[i].x, xu[i].y, xu[i].z, xu[i].w};
#pragma unroll
            for (int r = 0; r < kWaveRanks; ++r) {
                const float av8[8] = {av[r][0].x, av[r][0].y, av[r][0].z, av[r][0].w,
                                      av[r][1].x, av[r][1].y, av[r][1].z, av[r][1].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][r] = __builtin_fmaf(bf16_lo(w[j]), av8[2 * j], acc[i][r]);
                    acc[i][r] = __builtin_fmaf(bf16_hi(w[j]), av8[2 * j + 1], acc[i][r]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kDownRows; ++i)
#pragma unroll
        for (int r = 0; r < kWaveRanks; ++r) {
            float v = acc[i][r];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
            if (lane == 0 && m0 + i < m_rows && r0 + r < rank)
                part[((long)slice * m_rows + m0 + i) * rank + r0 + r] = v;
        }
}

template <bool F32, int ROWS>
__global__ __launch_bounds__(256) void lora_up_kernel(const float* __restrict__ part, const float* __restrict__ b,
                                                      void* __restrict__ y, int m_rows, int n_rows, int rank,
                                                      int slices, float scale) {
#pragma clang fp contract(off)
    const int n0 = (int)blockIdx.x * 256;
    const int n = n0 + (int)threadIdx.x;
    const int m0 = (int)blockIdx.y * ROWS;
    const int rows = m_rows - m0 < ROWS ? m_rows - m0 : ROWS;
    __shared__ float ts[ROWS][kRankBlock];
    __shared__ float bs[256][kRankBlock + 1];  // +1: thread n reads row n without bank conflicts
    float d[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; ++i) d[i] = 0.f;
    for (int r0 = 0; r0 < rank; r0 += kRankBlock) {
        const int rb = rank - r0 < kRankBlock ? rank - r0 : kRankBlock;
        __syncthreads();  // the previous block's values have been read
        for (int e = (int)threadIdx.x; e < ROWS * kRankBlock; e += 256) {
            const int i = e / kRankBlock, r = e % kRankBlock;
            float v = 0.f;
            if (i < rows && r < rb)
                for (int sl = 0; sl < slices; ++sl) v += part[((long)sl * m_rows + m0 + i) * rank + r0 + r];
            ts[i][r] = v;
        }
        // the workgroup's 256 rows of B, ranks r0 .. r0 + rb: consecutive threads read
        // consecutive ranks of a row (contiguous when rank == 16)
#pragma unroll
        for (int j = 0; j < kRankBlock; ++j) {
            const int e = j * 256 + (int)threadIdx.x;
            const int row = e / kRankBlock, r = e % kRankBlock;
            const int nn = n0 + row < n_rows ? n0 + row : n_rows - 1;  // rows of B past N: never used
            bs[row][r] = r < rb ? b[(long)nn * rank + r0 + r] : 0.f;
        }
        __syncthreads();
        float bv[kRankBlock];
#pragma unroll
        for (int r = 0; r < kRankBlock; ++r) bv[r] = bs[threadIdx.x][r];
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
#pragma unroll
            for (int r = 0; r < kRankBlock; ++r) d[i] = __builtin_fmaf(ts[i][r], bv[r], d[i]);
    }
    if (n >= n_rows) return;
    // every row's base value first (independent loads, one round trip), then the stores
    float base[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
        const long o = (long)(m0 + i) * n_rows + n;
        if (i < rows)
            base[i] = F32 ? static_cast<const float*>(y)[o]
                          : __uint_as_float((uint32_t)static_cast<const uint16_t*>(y)[o] << 16);
    }
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
        const long o = (long)(m0 + i) * n_rows + n;
        if (i < rows) {
            if (F32)
                static_cast<float*>(y)[o] = base[i] + d[i] * scale;
            else
                static_cast<uint16_t*>(y)[o] = f32_to_bf16(base[i] + round_bf16(d[i] * round_bf16(scale)));
        }
    }
}

}  // namespace

int lora_slices(int k) {
    const int chunks = k / 8;
    return chunks >= kLoraSlices * 64 ? kLoraSlices : (chunks + 63) / 64;
}

hipError_t launch_lora(const uint16_t* x, const float* a, const float* b, float* part, void* y, int m, int n, int k,
                       int rank, float scale, bool out_f32, hipStream_t stream) {
    static_assert(kWaveRanks * 4 == kRankBlock, "four waves per lora_down workgroup");
    const int slices = lora_slices(k);
    const int slice_chunks = (k / 8 + slices - 1) / slices;
    const dim3 dgrid((unsigned)((m + kDownRows - 1) / kDownRows), (unsigned)((rank + kRankBlock - 1) / kRankBlock),
                     (unsigned)slices);
    hipLaunchKernelGGL(lora_down_kernel, dgrid, dim3(256), 0, stream, x, a, part, m, rank, k, slice_chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // 16 rows per workgroup for decode-sized M, 64 (B read a quarter as often) beyond
    const int rows = m <= kUpRows ? kUpRows : kUpRowsLarge;
    const dim3 ugrid((unsigned)((n + 255) / 256), (unsigned)((m + rows - 1) / rows));
#define Q4_LORA_UP(F, R) \
    hipLaunchKernelGGL((lora_up_kernel<F, R>), ugrid, dim3(256), 0, stream, part, b, y, m, n, rank, slices, scale)
    if (out_f32) {
        if (rows == kUpRows) Q4_LORA_UP(true, kUpRows); else Q4_LORA_UP(true, kUpRowsLarge);
    } else {
        if (rows == kUpRows) Q4_LORA_UP(false, kUpRows); else Q4_LORA_UP(false, kUpRowsLarge);
    }
#undef Q4_LORA_UP
    return hipGetLastError();
}

}  // namespace q4
