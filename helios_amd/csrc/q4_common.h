// Shared device definitions for the gfx950 affine-Q4 kernels.
//
// Tiled weight layout (built once per projection by q4_layout.hip, resident in HBM):
//
//   A row block is 16 output rows (the N side of one 16x16x32 MFMA tile); a group
//   pair is 128 K values (two 64-wide quantization groups).  For row block rb and
//   group pair gp the packed nibbles form one 1 KiB tile, 16 bytes per lane:
//
//     tiles [NB][GP][64 lanes] of uint4
//     lane l -> row n = 16*rb + (l % 16), k-quarter kq = l / 16
//     .x = word(g=2gp,   half 0)   .y = word(g=2gp,   half 1)
//     .z = word(g=2gp+1, half 0)   .w = word(g=2gp+1, half 1)
//     word(g, h) holds q[n, 64g + 32h + 8kq + i], i = 0..7
//
//   so one coalesced dwordx4 load per lane fetches exactly the B operands of the
//   four 16x16x32 MFMAs that cover the group pair, with no LDS staging.
//
//   Within a word the eight nibbles are placed so that element pairs (2p, 2p+1)
//   come out as two bf16 values with two VALU ops:
//     rotr(word, 4p) has q[2p] in bits 3..6 and q[2p+1] in bits 19..22,
//     (rotr(word, 4p) & 0x00780078) | 0x3F803F80  ==  bf16x2(1 + q[2p]/16, 1 + q[2p+1]/16)
//   The values 1 + q/16 are exact in bf16, and the MFMA products with bf16 x are
//   exact in fp32, so the only rounding is fp32 accumulation.
//
//   Scales and biases sit beside the tiles, one uint2 per (rb, gp, row):
//     sb [NB][GP][16] of uint2, .x = s | b << 16 for group 2gp, .y for group 2gp+1
//
//   Padding: rows >= N and groups >= K/64 hold q = 0, s = 0, b = 0, so they add 0.
//
// Arithmetic (per group g, with X_g = sum of x over the group's 64 columns):
//   y += s*sum(x*q) + b*X_g = 16*s * (sum(x*(1+q/16)) - X_g) + b*X_g
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q4 {

constexpr int kGroup = 64;       // quantization group along K
constexpr int kRowBlock = 16;    // output rows per tile (MFMA N)
constexpr int kPairK = 128;      // K per group pair
constexpr uint32_t kOneBf16x2 = 0x3F803F80u;
constexpr uint32_t kNibMask = 0x00780078u;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Streaming loads of data read exactly once (weights): non-temporal hint.
__device__ __forceinline__ uint4 stream_load(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 stream_load(const uint2* p) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return make_uint2(v.x, v.y);
}

// Raw buffer loads: an offset at or beyond num_records reads as zero with no memory
// traffic, which replaces per-lane branches around loads (gfx9 resource word 3).
// Every buffer resource covers at most kMaxBufferBytes, so kOutOfRange is always
// past num_records (the host refuses larger buffers).
constexpr int kBufferFlags = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr size_t kMaxBufferBytes = (size_t)1 << 31;
constexpr int kNonTemporal = 2;  // aux bit 1: nt

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferFlags);
}

template <int AUX = 0>
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int AUX = 0>
__device__ __forceinline__ uint2 buffer_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, AUX);
    return make_uint2(v.x, v.y);
}

// (a & m) | c in one VALU op (gfx950 v_bitop3_b32, truth table 0xEA).  A builtin,
// not inline asm: the compiler's hazard recognizer must see this VALU write, since
// it often lands next to MFMAs whose operands are still being read.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, m, c, 0xEA);
}

__device__ __forceinline__ uint32_t rotr(uint32_t u, int s) {
    return __builtin_amdgcn_alignbit(u, u, s);
}

// Eight nibbles of one tiled word -> eight bf16 values 1 + q/16 in element order.
__device__ __forceinline__ bf16x8 expand_word(uint32_t u) {
    const uint32_t one = kOneBf16x2;
    uint4 d;
    d.x = and_or(u, kNibMask, one);
    d.y = and_or(rotr(u, 4), kNibMask, one);
    d.z = and_or(rotr(u, 8), kNibMask, one);
    d.w = and_or(rotr(u, 12), kNibMask, one);
    return __builtin_bit_cast(bf16x8, d);
}

// q[2p] and q[2p+1] of a tiled word, for the dequantize kernel.
__device__ __forceinline__ uint32_t word_nibble(uint32_t u, int i) {
    const uint32_t r = rotr(u, 4 * (i >> 1));
    return (i & 1) ? ((r >> 19) & 0xFu) : ((r >> 3) & 0xFu);
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace q4
