// LoRA delta on a quantized projection's output (native_model.cc:316-328):
//   y = model_dtype(base + model_dtype((float32(x) . A^T) . B^T * scale))
// A [rank, K] and B [N, rank] are fp32 (the adapter's tensors cast to float32,
// native_model.cc:3420-3426).  Two passes after the base qmm, which has already
// written base (bf16 in the bf16 model dtype, else fp32) into y:
//   lora_down: t[m, r] = sum_k x[m, k] A[r, k]     (fp32 accumulation)
//   lora_up:   y[m, n] = y[m, n] + delta,  delta = (sum_r t[m, r] B[n, r]) * scale
// In bf16 the scale is bf16 (model_scalar) and delta is rounded to bf16 before the
// bf16 add, as the reference's array ops round.
//
// lora_down: on the matrix cores from A's bf16 high and low parts (below); K is cut
// into lora_slices(k, m) slices (up to 8) until the workgroups fill the CUs, each
// writing its partial sums to part[slice][m][r].  No atomics: lora_up (or the GEMM's
// LoRA epilogue) adds the slices in a fixed order.
// lora_up: a 256-thread workgroup per (256 columns, 16 or 32 rows); t[m, r] (the
// slices summed in order, all of them requested at once) and the workgroup's rows of
// B are staged in LDS 16 ranks at a time (B with coalesced loads), and each thread
// takes its column's B values into registers and forms its rows' deltas.  With 32
// rows (M > 16) the deltas go through LDS and y is read and written in 16-byte pieces
// by consecutive threads (when N and y allow it); with 16 each thread updates its own
// column.  B is read once per 16 or 32 rows, y once.  Up to 4 rows with rank up to
// 64, lora_fused_kernel_f does both steps in one launch (below).
#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

constexpr int kDownWaves = 4;   // waves per lora_down workgroup (16 rows x 16 ranks x one slice of K)
constexpr int kRankBlock = 16;  // ranks per lora_up register block
constexpr int kUpRows = 16;     // rows of y per lora_up workgroup (M <= 16)
constexpr int kUpRowsLarge = 32;  // rows of y per lora_up workgroup (M > 16)
constexpr int kFusedRows = 4;      // M up to this with rank up to kFusedMaxRank: one fused launch
constexpr int kFusedMaxRank = 64;

// lora_down on the matrix cores: A is held as bf16 high and low parts [rank_pad][K]
// (A = Ah + Al to about 2^-17 relative, split once when the adapter is created), x is
// bf16, so t = x . Ah^T + x . Al^T is two 16x16x32 MFMAs per 32 columns of K with exact
// products and fp32 accumulation: within about 2^-17 of the fp32 product.  A 4-wave
// workgroup per (16 rows of x, 16 ranks, slice of K): the waves split the slice's
// 32-column steps, then their sums are added in wave order and written to
// part[slice][m][r].  Each lane reads 16 contiguous bytes of x (row l%16) and of Ah and
// Al (rank l%16) per step, so x is read once per 16 ranks.
__global__ __launch_bounds__(256) void lora_down_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ ah,
                                                        const uint16_t* __restrict__ al, float* __restrict__ part,
                                                        int m_rows, int rank, int k, int slice_steps) {
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int col = lane & 15, kq = lane >> 4;
    const int steps = k >> 5;
    const int s0 = (int)blockIdx.z * slice_steps;
    const int left = steps - s0;
    const int n_s = left < 0 ? 0 : left < slice_steps ? left : slice_steps;
    const int w0 = s0 + wave * n_s / kDownWaves, w1 = s0 + (wave + 1) * n_s / kDownWaves;
    const int m = (int)blockIdx.x * 16 + col;
    const int r = (int)blockIdx.y * 16 + col;  // rows of Ah / Al past rank are zero
    const uint16_t* xp = x + (long)(m < m_rows ? m : m_rows - 1) * k + 8 * kq;  // rows past M: never stored
    const uint16_t* hp = ah + (long)r * k + 8 * kq;
    const uint16_t* lp = al + (long)r * k + 8 * kq;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // the steps' loads go out in batches of kBatch before their MFMAs (a wave has one
    // or two batches, so one or two round trips instead of one per few steps; steps
    // past the wave's range reload its last step and skip the MFMAs)
    constexpr int kBatch = 8;
    for (int st0 = w0; st0 < w1; st0 += kBatch) {
        uint4 xv[kBatch], hv[kBatch], lv[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int st = st0 + i < w1 ? st0 + i : w1 - 1;
            xv[i] = *reinterpret_cast<const uint4*>(xp + 32 * st);
            hv[i] = *reinterpret_cast<const uint4*>(hp + 32 * st);
            lv[i] = *reinterpret_cast<const uint4*>(lp + 32 * st);
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            if (st0 + i < w1) {
                const bf16x8 xa = __builtin_bit_cast(bf16x8, xv[i]);
                acc = mfma16x16x32(xa, __builtin_bit_cast(bf16x8, hv[i]), acc);
                acc = mfma16x16x32(xa, __builtin_bit_cast(bf16x8, lv[i]), acc);
            }
        }
    }
    __shared__ f32x4 red[kDownWaves][64];
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4 v = red[0][lane];
#pragma unroll
    for (int w = 1; w < kDownWaves; ++w) {
        const f32x4 u = red[w][lane];
        v[0] += u[0];
        v[1] += u[1];
        v[2] += u[2];
        v[3] += u[3];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = (int)blockIdx.x * 16 + 4 * kq + e;
        if (row < m_rows && r < rank) part[((long)blockIdx.z * m_rows + row) * rank + r] = v[e];
    }
}

template <bool F32, int ROWS>
__global__ __launch_bounds__(256) void lora_up_kernel(const float* __restrict__ part, const float* __restrict__ b,
                                                      void* __restrict__ y, int m_rows, int n_rows, int rank,
                                                      int slices, float scale) {
#pragma clang fp contract(off)
    constexpr bool kStaged = ROWS > kUpRows;   // large M: y updated in 16-byte pieces
    constexpr int kPer = F32 ? 4 : 8;           // outputs per 16 bytes
    constexpr int kChunks = 256 / kPer;         // 16-byte pieces per tile row
    constexpr int kPieces = kStaged ? ROWS * kChunks / 256 : 1;  // y pieces per thread
    constexpr int kEntries = ROWS * kRankBlock / 256;          // t entries staged per thread
    static_assert(ROWS * kRankBlock % 256 == 0 && ROWS * kChunks % 256 == 0, "whole pieces per thread");
    const int n0 = (int)blockIdx.x * 256;
    const int n = n0 + (int)threadIdx.x;
    const int m0 = (int)blockIdx.y * ROWS;
    const int rows = m_rows - m0 < ROWS ? m_rows - m0 : ROWS;
    const bool vec = kStaged && n_rows % kPer == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    __shared__ float ts[ROWS][kRankBlock];
    __shared__ float bs[256][kRankBlock + 1];  // +1: thread n reads row n without bank conflicts
    __shared__ float dt[kStaged ? ROWS : 1][kStaged ? 256 + 4 : 1];  // the tile's deltas
    float d[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; ++i) d[i] = 0.f;
    // small M: y's current values, requested after the first rank block's operands
    // (loads return in order) so that they arrive while the deltas are formed; large
    // M reads them after the deltas (holding them across the math costs occupancy)
    float base[ROWS];
    for (int r0 = 0; r0 < rank; r0 += kRankBlock) {
        const int rb = rank - r0 < kRankBlock ? rank - r0 : kRankBlock;
        // this block's operands into registers: t (every slice of each entry at once)
        // and the workgroup's 256 rows of B (consecutive threads read consecutive ranks
        // of a row: contiguous when rank == 16)
        float pv[kEntries][kLoraSlices];
#pragma unroll
        for (int u = 0; u < kEntries; ++u) {
            const int e = u * 256 + (int)threadIdx.x;
            const int i = e / kRankBlock, r = e % kRankBlock;
            const bool live = i < rows && r < rb;
#pragma unroll
            for (int sl = 0; sl < kLoraSlices; ++sl)
                pv[u][sl] = live && sl < slices ? part[((long)sl * m_rows + m0 + i) * rank + r0 + r] : 0.f;
        }
        float bl[kRankBlock];
#pragma unroll
        for (int j = 0; j < kRankBlock; ++j) {
            const int e = j * 256 + (int)threadIdx.x;
            const int row = e / kRankBlock, r = e % kRankBlock;
            const int nn = n0 + row < n_rows ? n0 + row : n_rows - 1;  // rows of B past N: never used
            bl[j] = r < rb ? b[(long)nn * rank + r0 + r] : 0.f;
        }
        if (r0 == 0) {
            if constexpr (!kStaged) {
#pragma unroll
                for (int i = 0; i < ROWS; ++i) {
                    const long o = (long)(m0 + i) * n_rows + n;
                    base[i] = i < rows && n < n_rows
                                  ? (F32 ? static_cast<const float*>(y)[o]
                                         : __uint_as_float((uint32_t)static_cast<const uint16_t*>(y)[o] << 16))
                                  : 0.f;
                }
            }
        }
        __syncthreads();  // the previous block's values have been read
#pragma unroll
        for (int u = 0; u < kEntries; ++u) {
            const int e = u * 256 + (int)threadIdx.x;
            float v = pv[u][0];  // summed in slice order
#pragma unroll
            for (int sl = 1; sl < kLoraSlices; ++sl)
                if (sl < slices) v += pv[u][sl];
            ts[e / kRankBlock][e % kRankBlock] = v;
        }
#pragma unroll
        for (int j = 0; j < kRankBlock; ++j) {
            const int e = j * 256 + (int)threadIdx.x;
            bs[e / kRankBlock][e % kRankBlock] = bl[j];
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
    if constexpr (kStaged) {
        if (vec) {
#pragma unroll
            for (int i = 0; i < ROWS; ++i) dt[i][threadIdx.x] = d[i];
            // consecutive threads take consecutive 16-byte pieces of a row; a piece lies
            // wholly inside or outside the row (N is a multiple of the piece); all of a
            // thread's pieces are requested before the first store
            uint4 ypre[kPieces];
#pragma unroll
            for (int u = 0; u < kPieces; ++u) {
                const int q = u * 256 + (int)threadIdx.x;
                const int i = q / kChunks, nn = n0 + (q % kChunks) * kPer;
                ypre[u] = i < rows && nn < n_rows
                              ? *reinterpret_cast<const uint4*>(static_cast<const char*>(y) +
                                                                ((long)(m0 + i) * n_rows + nn) * (F32 ? 4 : 2))
                              : make_uint4(0, 0, 0, 0);
            }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < kPieces; ++u) {
                const int q = u * 256 + (int)threadIdx.x;
                const int i = q / kChunks, j = q % kChunks;
                const int nn = n0 + j * kPer;
                if (i >= rows || nn >= n_rows) continue;
                const long o = (long)(m0 + i) * n_rows + nn;
                const float* dv = &dt[i][j * kPer];
                if constexpr (F32) {
                    float4 v = __builtin_bit_cast(float4, ypre[u]);
                    v.x = v.x + dv[0] * scale;
                    v.y = v.y + dv[1] * scale;
                    v.z = v.z + dv[2] * scale;
                    v.w = v.w + dv[3] * scale;
                    *reinterpret_cast<float4*>(static_cast<float*>(y) + o) = v;
                } else {
                    const uint32_t w[4] = {ypre[u].x, ypre[u].y, ypre[u].z, ypre[u].w};
                    const float sc = round_bf16(scale);
                    uint32_t out[4];
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const uint32_t lo = f32_to_bf16(bf16_lo(w[h]) + round_bf16(dv[2 * h] * sc));
                        const uint32_t hi = f32_to_bf16(bf16_hi(w[h]) + round_bf16(dv[2 * h + 1] * sc));
                        out[h] = lo | (hi << 16);
                    }
                    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(y) + o) = make_uint4(out[0], out[1], out[2], out[3]);
                }
            }
            return;
        }
    }
    if (n >= n_rows) return;
    if constexpr (kStaged) {  // N or y not 16-byte friendly: every row's value now, then the stores
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const long o = (long)(m0 + i) * n_rows + n;
            base[i] = i < rows ? (F32 ? static_cast<const float*>(y)[o]
                                      : __uint_as_float((uint32_t)static_cast<const uint16_t*>(y)[o] << 16))
                               : 0.f;
        }
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


// Small M (lora_fused(m, rank)): the whole delta in one launch, with no scratch.  A
// 1024-thread workgroup per 256 columns of y:
//   (1) t = x . A^T for all rows and ranks, computed by every workgroup (x and A come
//       from L2 after the first): the 16 waves take 16 ranks of a block, a wave's
//       lanes interleave K's 8-column chunks, and each wave sums its lanes by
//       shuffles (a fixed order) into LDS;
//   (2) each column's delta from t and its row of B, four threads per column with a
//       contiguous quarter of the ranks each, the quarters added in a fixed order in
//       LDS, then y updated as lora_up does.
__global__ __launch_bounds__(1024) void lora_fused_kernel_f(const uint16_t* __restrict__ x, const float* __restrict__ a,
                                                            const float* __restrict__ b, void* __restrict__ y,
                                                            int m_rows, int n_rows, int k, int rank, float scale,
                                                            int out_f32) {
#pragma clang fp contract(off)
    __shared__ float ts[kFusedRows][kFusedMaxRank];
    __shared__ float dq[4][kFusedRows][256];
    const int tid = (int)threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int chunks = k >> 3;
    for (int r0 = 0; r0 < rank; r0 += 16) {
        const int r = r0 + wave;
        float acc[kFusedRows];
#pragma unroll
        for (int i = 0; i < kFusedRows; ++i) acc[i] = 0.f;
        if (r < rank) {
            const float* ar = a + (long)r * k;
#pragma unroll 2
            for (int c = lane; c < chunks; c += 64) {
                const float4 a0 = *reinterpret_cast<const float4*>(ar + 8 * c);
                const float4 a1 = *reinterpret_cast<const float4*>(ar + 8 * c + 4);
                const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                for (int i = 0; i < kFusedRows; ++i) {
                    if (i < m_rows) {
                        const uint4 xu = *reinterpret_cast<const uint4*>(x + (long)i * k + 8 * c);
                        const uint32_t w[4] = {xu.x, xu.y, xu.z, xu.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            acc[i] = __builtin_fmaf(bf16_lo(w[j]), av[2 * j], acc[i]);
                            acc[i] = __builtin_fmaf(bf16_hi(w[j]), av[2 * j + 1], acc[i]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kFusedRows; ++i) {
            float v = acc[i];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
            if (lane == 0 && r < rank) ts[i][r] = v;
        }
    }
    __syncthreads();
    const int col = tid & 255, q = tid >> 8;
    const int n = (int)blockIdx.x * 256 + col;
    const int r_lo = q * rank / 4, r_hi = (q + 1) * rank / 4;
    float d[kFusedRows];
#pragma unroll
    for (int i = 0; i < kFusedRows; ++i) d[i] = 0.f;
    if (n < n_rows) {
        const float* br = b + (long)n * rank;
        for (int r = r_lo; r < r_hi; ++r) {
            const float bv = br[r];
#pragma unroll
            for (int i = 0; i < kFusedRows; ++i) d[i] = __builtin_fmaf(ts[i][r], bv, d[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < kFusedRows; ++i) dq[q][i][col] = d[i];
    __syncthreads();
    if (q != 0 || n >= n_rows) return;
    for (int i = 0; i < m_rows; ++i) {
        const float v = ((dq[0][i][col] + dq[1][i][col]) + dq[2][i][col]) + dq[3][i][col];
        const long o = (long)i * n_rows + n;
        if (out_f32) {
            static_cast<float*>(y)[o] = static_cast<const float*>(y)[o] + v * scale;
        } else {
            const float base = __uint_as_float((uint32_t)static_cast<const uint16_t*>(y)[o] << 16);
            static_cast<uint16_t*>(y)[o] = f32_to_bf16(base + round_bf16(v * round_bf16(scale)));
        }
    }
}

}  // namespace

int lora_slices(int k, int m) {
    // slices of K until the (16-row block, slice) workgroups fill the CUs, each wave
    // keeping at least four 32-column steps
    const int steps = k / 32;
    const int wgs = (m + 15) / 16;
    int s = 1;
    while (s < kLoraSlices && wgs * s < 256 && steps / (2 * s * kDownWaves) >= 4) s *= 2;
    return s;
}

bool lora_fused(int m, int rank) { return m <= kFusedRows && rank <= kFusedMaxRank; }

hipError_t launch_lora_down(const uint16_t* x, const uint16_t* a_hi, const uint16_t* a_lo, float* part, int m,
                            int k, int rank, hipStream_t stream) {
    const int slices = lora_slices(k, m);
    const int slice_steps = (k / 32 + slices - 1) / slices;
    const dim3 dgrid((unsigned)((m + 15) / 16), (unsigned)((rank + 15) / 16), (unsigned)slices);
    hipLaunchKernelGGL(lora_down_kernel, dgrid, dim3(64 * kDownWaves), 0, stream, x, a_hi, a_lo, part, m, rank, k,
                       slice_steps);
    return hipGetLastError();
}

hipError_t launch_lora(const uint16_t* x, const float* a, const uint16_t* a_hi, const uint16_t* a_lo, const float* b,
                       float* part, void* y, int m, int n, int k, int rank, float scale, bool out_f32,
                       hipStream_t stream) {
    if (lora_fused(m, rank)) {
        hipLaunchKernelGGL(lora_fused_kernel_f, dim3((unsigned)((n + 255) / 256)), dim3(1024), 0, stream, x, a, b, y, m,
                           n, k, rank, scale, out_f32 ? 1 : 0);
        return hipGetLastError();
    }
    const int slices = lora_slices(k, m);
    hipError_t e = launch_lora_down(x, a_hi, a_lo, part, m, k, rank, stream);
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
