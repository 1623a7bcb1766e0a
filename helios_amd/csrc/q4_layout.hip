// Weight-layout kernels: MLX affine layout -> tiled MFMA layout (one projection, or a
// gate|up pair interleaved 8 rows at a time), and the bit-exact fp32 dequantize of
// the tiled layout (the check that the tiles hold every bit).
#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

// MLX word (q[i] at bits 4i) -> tiled word (see q4_common.h): pairs (2p, 2p+1) go to
// bits (4p, 16+4p), then the word is rotated left by 3.
__device__ __forceinline__ uint32_t tile_word(uint32_t u) {
    uint32_t t = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        t |= ((u >> (8 * p)) & 0xFu) << (4 * p);
        t |= ((u >> (8 * p + 4)) & 0xFu) << (16 + 4 * p);
    }
    return (t << 3) | (t >> 29);
}

// Source row of tiled row 16*rb + c: row 16*rb + c of the projection, or for a
// gate|up pair (pair_rows = F > 0) row 8*rb + c%8 of gate (c < 8) or of up (c >= 8).
struct SourceRow {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    int row;
    bool valid;
};

__device__ __forceinline__ SourceRow source_row(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                                const uint32_t* w2, const uint16_t* s2, const uint16_t* b2,
                                                long rb, int c, int n_rows, int pair_rows) {
    if (pair_rows > 0) {
        const int row = (int)(rb * 8 + (c & 7));
        return c < 8 ? SourceRow{w, s, b, row, row < pair_rows} : SourceRow{w2, s2, b2, row, row < pair_rows};
    }
    const int row = (int)(rb * 16 + c);
    return SourceRow{w, s, b, row, row < n_rows};
}

__global__ void repack_kernel(const uint32_t* __restrict__ w_a, const uint16_t* __restrict__ s_a,
                              const uint16_t* __restrict__ b_a, const uint32_t* __restrict__ w_b,
                              const uint16_t* __restrict__ s_b, const uint16_t* __restrict__ b_b,
                              uint4* __restrict__ tiles, uint2* __restrict__ sb, int n_rows, int pair_rows, int k,
                              int groups, int gpairs, long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int lane = (int)(tid & 63);
    const long t = tid >> 6;
    const int gp = (int)(t % gpairs);
    const long rb = t / gpairs;
    const SourceRow src = source_row(w_a, s_a, b_a, w_b, s_b, b_b, rb, lane & 15, n_rows, pair_rows);
    const uint32_t* w = src.w;
    const uint16_t* s = src.s;
    const uint16_t* b = src.b;
    const int row = src.row;
    const int kq = lane >> 4;
    const int words_per_row = k / 8;
    uint32_t out[4];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = 2 * gp + gi;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t u = 0;
            if (src.valid && g < groups) u = w[(long)row * words_per_row + 8 * g + 4 * h + kq];
            out[2 * gi + h] = tile_word(u);
        }
    }
    tiles[tid] = make_uint4(out[0], out[1], out[2], out[3]);
    if (kq == 0) {
        uint32_t v[2];
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
            const int g = 2 * gp + gi;
            v[gi] = 0;
            if (src.valid && g < groups) {
                const long idx = (long)row * groups + g;
                v[gi] = (uint32_t)s[idx] | ((uint32_t)b[idx] << 16);
            }
        }
        sb[t * 16 + (lane & 15)] = make_uint2(v[0], v[1]);
    }
}

// out row of tiled row 16*rb + c: the same row, or for a gate|up pair gate row r at
// out row r and up row r at out row F + r (out is [2, F, K])
__global__ void dequantize_kernel(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                                  float* __restrict__ out, int n_rows, int pair_rows, int k, int groups, int gpairs,
                                  long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int lane = (int)(tid & 63);
    const long t = tid >> 6;
    const int gp = (int)(t % gpairs);
    const long rb = t / gpairs;
    const int c = lane & 15;
    const int kq = lane >> 4;
    int row;
    if (pair_rows > 0) {
        const int r = (int)(rb * 8 + (c & 7));
        if (r >= pair_rows) return;
        row = c < 8 ? r : pair_rows + r;
    } else {
        row = (int)(rb * 16 + c);
        if (row >= n_rows) return;
    }
    const uint4 wv = tiles[tid];
    const uint2 sv = sb[t * 16 + (lane & 15)];
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = 2 * gp + gi;
        if (g >= groups) continue;
        const uint32_t sbv = gi ? sv.y : sv.x;
        const float sc = bf16_lo(sbv);
        const float bi = bf16_hi(sbv);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t u = words[2 * gi + h];
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sc, (float)word_nibble(u, i), bi);
            float4* dst = reinterpret_cast<float4*>(out + (long)row * k + 64 * g + 32 * h + 8 * kq);
            dst[0] = make_float4(v[0], v[1], v[2], v[3]);
            dst[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
}

// Row gather of the dequantized weight: out[t, :] = W[ids[t], :] (fp32, or bf16 rounded
// once).  One thread per (token, group pair, k-quarter): the four words of lane
// (ids[t] % 16, kq) in tile (ids[t] / 16, gp), 32 values.  ids outside [0, n_rows)
// give zero rows.
__global__ void embed_kernel(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                             const int32_t* __restrict__ ids, void* __restrict__ out, int out_f32, int n_rows, int k,
                             int groups, int gpairs, long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int kq = (int)(tid & 3);
    const long r = tid >> 2;
    const int gp = (int)(r % gpairs);
    const long t = r / gpairs;
    const int id = ids[t];
    const bool valid = id >= 0 && id < n_rows;
    const long rb = valid ? id >> 4 : 0;
    const int col = valid ? id & 15 : 0;
    const long tile = rb * gpairs + gp;
    const uint4 wv = valid ? tiles[tile * 64 + col + 16 * kq] : make_uint4(0, 0, 0, 0);
    const uint2 sv = valid ? sb[tile * 16 + col] : make_uint2(0, 0);
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = 2 * gp + gi;
        if (g >= groups) continue;
        const uint32_t sbv = gi ? sv.y : sv.x;
        const float sc = bf16_lo(sbv);
        const float bi = bf16_hi(sbv);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sc, (float)word_nibble(words[2 * gi + h], i), bi);
            const long o = t * k + 64 * g + 32 * h + 8 * kq;
            if (out_f32) {
                float4* dst = reinterpret_cast<float4*>(static_cast<float*>(out) + o);
                dst[0] = make_float4(v[0], v[1], v[2], v[3]);
                dst[1] = make_float4(v[4], v[5], v[6], v[7]);
            } else {
                uint32_t p[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    p[j] = (uint32_t)f32_to_bf16(v[2 * j]) | ((uint32_t)f32_to_bf16(v[2 * j + 1]) << 16);
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + o) = make_uint4(p[0], p[1], p[2], p[3]);
            }
        }
    }
}

}  // namespace

hipError_t launch_embed(const uint4* tiles, const uint2* sb, const int32_t* ids, int count, void* out, bool out_f32,
                        const Layout& l, hipStream_t stream) {
    const long total = (long)count * l.gp * 4;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)grid), dim3(block), 0, stream, tiles, sb, ids, out, out_f32 ? 1 : 0,
                       l.n, l.k, l.g, l.gp, total);
    return hipGetLastError();
}

hipError_t launch_repack(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint32_t* w_up,
                         const uint16_t* s_up, const uint16_t* b_up, uint4* tiles, uint2* sb, const Layout& l,
                         int pair_rows, hipStream_t stream) {
    const long total = (long)l.nb * l.gp * 64;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)grid), dim3(block), 0, stream, w, s, b, w_up, s_up, b_up, tiles,
                       sb, l.n, pair_rows, l.k, l.g, l.gp, total);
    return hipGetLastError();
}

hipError_t launch_dequantize(const uint4* tiles, const uint2* sb, float* out, const Layout& l, int pair_rows,
                             hipStream_t stream) {
    const long total = (long)l.nb * l.gp * 64;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)grid), dim3(block), 0, stream, tiles, sb, out,
                       l.n, pair_rows, l.k, l.g, l.gp, total);
    return hipGetLastError();
}

}  // namespace q4
