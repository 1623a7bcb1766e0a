// Weight-layout kernels: MLX affine layout -> tiled MFMA layout (one projection, or a
// gate|up pair interleaved 8 rows at a time) as records of tiled words and scale/bias
// words (q4_kernels.h), and the bit-exact fp32 dequantize of the records (the check
// that they hold every bit).
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
    tiles[t * kRecU4 + lane] = make_uint4(out[0], out[1], out[2], out[3]);
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
        sb[t * kRecU2 + (lane & 15)] = make_uint2(v[0], v[1]);
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
    const uint4 wv = tiles[t * kRecU4 + lane];
    const uint2 sv = sb[t * kRecU2 + (lane & 15)];
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
    const uint4 wv = valid ? tiles[tile * kRecU4 + col + 16 * kq] : make_uint4(0, 0, 0, 0);
    const uint2 sv = valid ? sb[tile * kRecU2 + col] : make_uint2(0, 0);
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

// ---------------------------------------------------------------------------
// 8-bit affine weights as two 4-bit planes
// ---------------------------------------------------------------------------
// An 8-bit code q = 16*qh + ql gives w = s*q + b = (16s)*qh + b + s*ql.  The handle
// stores the projection as a 4-bit one over K' = 2K: groups [0, G) hold the high
// nibbles with scale 16s and bias b, groups [G, 2G) the low nibbles with scale s and
// bias 0 (16s is exact in bf16), and the input is x' = [x | x].  Every 4-bit kernel
// then computes y = x' . W'^T = x . W^T with the same exact products.
//
// MLX 8-bit words hold four codes, lowest byte first (code k in word k/4).

// Four-bit word (MLX nibble order) of plane `hi` for codes c0..c7 = two 8-bit words.
__device__ __forceinline__ uint32_t plane_word(uint32_t w0, uint32_t w1, bool hi) {
    uint32_t u = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t byte = ((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xFFu;
        u |= (hi ? byte >> 4 : byte & 0xFu) << (4 * i);
    }
    return u;
}

__global__ void repack8_kernel(const uint32_t* __restrict__ w_a, const uint16_t* __restrict__ s_a,
                               const uint16_t* __restrict__ b_a, const uint32_t* __restrict__ w_b,
                               const uint16_t* __restrict__ s_b, const uint16_t* __restrict__ b_b,
                               uint4* __restrict__ tiles, uint2* __restrict__ sb, int n_rows, int pair_rows, int k8,
                               int groups8, int gpairs, long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int lane = (int)(tid & 63);
    const long t = tid >> 6;
    const int gp = (int)(t % gpairs);
    const long rb = t / gpairs;
    const SourceRow src = source_row(w_a, s_a, b_a, w_b, s_b, b_b, rb, lane & 15, n_rows, pair_rows);
    const int kq = lane >> 4;
    const int words_per_row = k8 / 4;
    uint32_t out[4];
    uint32_t sbw[2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int gq = 2 * gp + gi;  // group of K'
        const bool live = src.valid && gq < 2 * groups8;
        const bool hi = gq < groups8;
        const int g = hi ? gq : gq - groups8;  // group of the 8-bit row
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t u = 0;
            if (live) {
                const long wi = (long)src.row * words_per_row + 16 * g + 8 * h + 2 * kq;
                u = plane_word(src.w[wi], src.w[wi + 1], hi);
            }
            out[2 * gi + h] = tile_word(u);
        }
        sbw[gi] = 0;
        if (live) {
            const long idx = (long)src.row * groups8 + g;
            const uint32_t sc = src.s[idx], bi = src.b[idx];
            // 16s is exact in bf16 (a power-of-two scaling; subnormal s included)
            const uint32_t sc16 = f32_to_bf16(bf16_lo(sc) * 16.0f);
            sbw[gi] = hi ? (sc16 | (bi << 16)) : sc;
        }
    }
    tiles[t * kRecU4 + lane] = make_uint4(out[0], out[1], out[2], out[3]);
    if (kq == 0) sb[t * kRecU2 + (lane & 15)] = make_uint2(sbw[0], sbw[1]);
}

// fp32 s*q + b of 8 codes of tiled row lane (col) for original group g and half h,
// from the two planes of a two-plane handle.
__device__ __forceinline__ void two_plane_values(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                                                 long rb, int gpairs, int groups8, int g, int h, int col, int kq,
                                                 float v[8]) {
    const int glo = groups8 + g;
    const long thi = rb * gpairs + (g >> 1), tlo = rb * gpairs + (glo >> 1);
    const uint4 whi = tiles[thi * kRecU4 + col + 16 * kq];
    const uint4 wlo = tiles[tlo * kRecU4 + col + 16 * kq];
    const uint32_t ahi[4] = {whi.x, whi.y, whi.z, whi.w};
    const uint32_t alo[4] = {wlo.x, wlo.y, wlo.z, wlo.w};
    const uint32_t uhi = ahi[2 * (g & 1) + h], ulo = alo[2 * (glo & 1) + h];
    const uint2 shi = sb[thi * kRecU2 + col], slo = sb[tlo * kRecU2 + col];
    const uint32_t sbh = (g & 1) ? shi.y : shi.x, sbl = (glo & 1) ? slo.y : slo.x;
    const float sc = bf16_lo(sbl);  // s (the low plane's scale)
    const float bi = bf16_hi(sbh);  // b (the high plane's bias)
#pragma unroll
    for (int i = 0; i < 8; ++i)
        v[i] = __builtin_fmaf(sc, (float)(16u * word_nibble(uhi, i) + word_nibble(ulo, i)), bi);
}

// dequantize of a two-plane handle: thread per (row block, original group, lane)
__global__ void dequantize8_kernel(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                                   float* __restrict__ out, int n_rows, int pair_rows, int k8, int groups8, int gpairs,
                                   long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int lane = (int)(tid & 63);
    const long t = tid >> 6;
    const int g = (int)(t % groups8);
    const long rb = t / groups8;
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
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float v[8];
        two_plane_values(tiles, sb, rb, gpairs, groups8, g, h, c, kq, v);
        float4* dst = reinterpret_cast<float4*>(out + (long)row * k8 + 64 * g + 32 * h + 8 * kq);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// embedding rows of a two-plane handle: thread per (token, original group, k-quarter)
__global__ void embed8_kernel(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                              const int32_t* __restrict__ ids, void* __restrict__ out, int out_f32, int n_rows, int k8,
                              int groups8, int gpairs, long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int kq = (int)(tid & 3);
    const long r = tid >> 2;
    const int g = (int)(r % groups8);
    const long t = r / groups8;
    const int id = ids[t];
    const bool valid = id >= 0 && id < n_rows;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (valid) two_plane_values(tiles, sb, id >> 4, gpairs, groups8, g, h, id & 15, kq, v);
        const long o = t * k8 + 64 * g + 32 * h + 8 * kq;
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

}  // namespace

hipError_t launch_repack8(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint32_t* w_up,
                          const uint16_t* s_up, const uint16_t* b_up, uint4* tiles, uint2* sb, const Layout& l,
                          int pair_rows, hipStream_t stream) {
    const long total = (long)l.nb * l.gp * 64;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    hipLaunchKernelGGL(repack8_kernel, dim3((unsigned)grid), dim3(block), 0, stream, w, s, b, w_up, s_up, b_up, tiles,
                       sb, l.n, pair_rows, l.k / 2, l.g / 2, l.gp, total);
    return hipGetLastError();
}

hipError_t launch_dequantize8(const uint4* tiles, const uint2* sb, float* out, const Layout& l, int pair_rows,
                              hipStream_t stream) {
    const long total = (long)l.nb * (l.g / 2) * 64;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    hipLaunchKernelGGL(dequantize8_kernel, dim3((unsigned)grid), dim3(block), 0, stream, tiles, sb, out, l.n, pair_rows,
                       l.k / 2, l.g / 2, l.gp, total);
    return hipGetLastError();
}

hipError_t launch_embed8(const uint4* tiles, const uint2* sb, const int32_t* ids, int count, void* out, bool out_f32,
                         const Layout& l, hipStream_t stream) {
    const long total = (long)count * (l.g / 2) * 4;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    hipLaunchKernelGGL(embed8_kernel, dim3((unsigned)grid), dim3(block), 0, stream, tiles, sb, ids, out,
                       out_f32 ? 1 : 0, l.n, l.k / 2, l.g / 2, l.gp, total);
    return hipGetLastError();
}

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
