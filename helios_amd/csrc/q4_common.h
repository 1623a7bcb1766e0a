// Shared device definitions for the gfx950 affine-Q4 kernels.
//
// Tiled weight layout (built once per projection by q4_layout.hip, resident in HBM):
//
//   A row block is 16 output rows (the N side of one 16x16x32 MFMA tile); a group
//   pair is 128 K values (two 64-wide quantization groups).  Row block rb and group
//   pair gp own one 1152-byte record (records [NB][GP]): a 1 KiB tile of the packed
//   nibbles, 16 bytes per lane, then the 16 rows' scale/bias words (below):
//
//     tile of record (rb, gp): 64 lanes of uint4
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
//   Scales and biases follow their tile in the record, one uint2 per row:
//     16 uint2, .x = s | b << 16 for group 2gp, .y for group 2gp+1
//   (a row block's run of records is then one contiguous stream of weight bytes)
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

// The same with a wave-uniform part of the offset in the instruction's scalar offset
// (soff: an SGPR, no VGPR spent on it).  In-range lanes keep off + soff inside the
// buffer; lanes at kOutOfRange read zero.
template <int AUX = 0>
__device__ __forceinline__ uint4 buffer_load16s(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, AUX);
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

// The GEMM's fp16 form.  q - 8 lies in [-8, 7] and a bf16 scale has an 8-bit
// significand, so s' (q - 8) has at most 11 significant bits (255 * 8 < 2^11): it is
// exact in fp16 whenever s' lies in [2^-14, 2^13) or is zero.  Eight nibbles of one
// tiled word -> the eight fp16 values s' (q - 8) in element order: the mask puts q in
// mantissa bits 3..6 under the exponent of 128, giving 128 + q; minus 136 is q - 8
// (exact), times s' (exact).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kF16x2Of128 = 0x58005800u;
__device__ __forceinline__ f16x8 expand_word_f16(uint32_t u, f16x2 s) {
    const f16x2 off = {(_Float16)-136.0f, (_Float16)-136.0f};
    f16x2 v[4];
    v[0] = __builtin_bit_cast(f16x2, and_or(u, kNibMask, kF16x2Of128));
    v[1] = __builtin_bit_cast(f16x2, and_or(rotr(u, 4), kNibMask, kF16x2Of128));
    v[2] = __builtin_bit_cast(f16x2, and_or(rotr(u, 8), kNibMask, kF16x2Of128));
    v[3] = __builtin_bit_cast(f16x2, and_or(rotr(u, 12), kNibMask, kF16x2Of128));
    f16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f16x2 w = (v[i] + off) * s;
        r[2 * i] = w[0];
        r[2 * i + 1] = w[1];
    }
    return r;
}

// 8-bit codes in one pass (a two-plane handle's GEMM): the high plane's word h and the
// low plane's word l of the same (lane, group, half) hold q >> 4 and q & 15 of the same
// eight codes.  -> the eight fp16 values 1024 + q (exact: 11 significant bits) in
// element order: q_h from bits 3..6 shifted to 4..7, q_l rotated down to bits 0..3,
// under the exponent of 1024.
constexpr uint32_t kF16x2Of1024 = 0x64006400u;
__device__ __forceinline__ f16x8 expand_word_q8(uint32_t h, uint32_t l) {
    uint4 d;
    d.x = ((h & kNibMask) << 1) | and_or(rotr(l, 3), 0x000F000Fu, kF16x2Of1024);
    d.y = ((rotr(h, 4) & kNibMask) << 1) | and_or(rotr(l, 7), 0x000F000Fu, kF16x2Of1024);
    d.z = ((rotr(h, 8) & kNibMask) << 1) | and_or(rotr(l, 11), 0x000F000Fu, kF16x2Of1024);
    d.w = ((rotr(h, 12) & kNibMask) << 1) | and_or(rotr(l, 15), 0x000F000Fu, kF16x2Of1024);
    return __builtin_bit_cast(f16x8, d);
}

// q[2p] and q[2p+1] of a tiled word, for the dequantize kernel.
__device__ __forceinline__ uint32_t word_nibble(uint32_t u, int i) {
    const uint32_t r = rotr(u, 4 * (i >> 1));
    return (i & 1) ? ((r >> 19) & 0xFu) : ((r >> 3) & 0xFu);
}

// Reductions over the eight lanes of an aligned octet (lanes 8i..8i+7) by DPP lane moves
// inside the wave, with no trip through the LDS crossbar (ds_bpermute, which is what
// __shfl_xor becomes): partners at distance 1 and 2 (quad permutes), then the other quad
// (row_half_mirror pairs lane j of the octet with lane 7 - j, which by then holds that
// quad's value).  Every lane ends with the result; the adds are those of the xor 1, 2, 4
// butterfly, in the same order, so the sums are the same bits.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppSwap1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppSwap2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
__device__ __forceinline__ uint32_t octet_max(uint32_t v) {
    uint32_t o = dpp_mov<kDppSwap1>(v);
    v = v > o ? v : o;
    o = dpp_mov<kDppSwap2>(v);
    v = v > o ? v : o;
    o = dpp_mov<kDppHalfMirror>(v);
    return v > o ? v : o;
}
__device__ __forceinline__ float octet_sum(float v) {
    v += __uint_as_float(dpp_mov<kDppSwap1>(__float_as_uint(v)));
    v += __uint_as_float(dpp_mov<kDppSwap2>(__float_as_uint(v)));
    v += __uint_as_float(dpp_mov<kDppHalfMirror>(__float_as_uint(v)));
    return v;
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet: the hardware conversion
// (v_cvt_pk_bf16_f32), branch-free.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// ---------------------------------------------------------------------------
// Output stage: plain projection (bf16 or fp32) or a gate|up pair with GeGLU
// ---------------------------------------------------------------------------
// A gate|up pair is tiled as one projection whose 16-row block j holds gate rows
// 8j..8j+7 in columns 0..7 and the same up rows in columns 8..15, so each output
// h[m, 8j + c] = geglu(gate, up) combines columns c and c + 8 of one block.
enum OutMode : int {
    kOutBf16 = 0,        // y bf16 [M, N]
    kOutF32 = 1,         // y fp32 [M, N] (also the split-K partial planes)
    kOutGegluBf16 = 2,   // h bf16 [M, F], the bf16 model dtype's GeGLU
    kOutGegluF32 = 3,    // h fp32 [M, F], the float32 override's GeGLU
    kOutGreedyBf16 = 4,  // lm_head: softcap in bf16 ops, optional logits, best (value, index) per block
    kOutGreedyF32 = 5,   // the same in fp32
    kOutLoraBf16 = 6,    // GEMM only: y bf16 = base + the LoRA delta (LoraEpilogue), bf16 ops
    kOutLoraF32 = 7,     // the same in fp32
};

// The LoRA delta a GEMM epilogue adds to its outputs (kOutLora*): t = x . A^T as
// `slices` fp32 partial planes [slices][M][rank] (summed in slice order), B [N][rank]
// fp32, the adapter's scale; rank a multiple of 4, at most 32.
struct LoraEpilogue {
    const float* part;
    const float* b;
    int rank;
    int slices;
    float scale;
};

// Where and how a decode kernel writes its outputs.
struct OutParams {
    void* y;                   // y [M, N], h [M, F], or the greedy modes' logits [M, N] (may be null)
    unsigned long long* part;  // greedy modes: best key of each (row, 16-row block), [M][nb]
    int mode;
    int n_out;                 // GeGLU modes: F
    int nb;                    // greedy modes: row blocks (the stride of part)
    float cap;                 // greedy modes: the softcap (0: none)
};

// Byte offset in x of 16-byte unit c of x' (rows of k elements), for x rows of kx
// elements: kx = k, or k / 2 for a two-plane 8-bit handle, whose x' = [x | x] repeats
// each row (column c of x' is column c mod kx of x).
__device__ __forceinline__ uint32_t xprime_offset(int c, int k, int kx) {
    if (kx == k) return (uint32_t)c * 16u;
    const int rowc = k >> 3, rowcx = kx >> 3;
    const int row = c / rowc;
    const int cr = c - row * rowc;
    return (uint32_t)(row * rowcx + (cr >= rowcx ? cr - rowcx : cr)) * 16u;
}

// Output parameters of the 16-row slab `slab` of a launch: y (or h, or the logits)
// and the greedy keys advance by 16 rows.  Decode kernels launched over M > 16 rows
// take their slab from blockIdx.y.
__device__ __forceinline__ OutParams slab_params(OutParams op, int slab, int n_rows) {
    const bool geglu = op.mode == kOutGegluBf16 || op.mode == kOutGegluF32;
    const bool f32 = op.mode == kOutF32 || op.mode == kOutGegluF32 || op.mode == kOutGreedyF32;
    const long row0 = 16L * slab;
    if (op.y != nullptr) op.y = static_cast<char*>(op.y) + row0 * (geglu ? op.n_out : n_rows) * (f32 ? 4 : 2);
    if (op.part != nullptr) op.part += row0 * op.nb;
    return op;
}

__device__ __forceinline__ float round_bf16(float v) { return (float)(__bf16)v; }

// GeGLU of native_model.cc:378-386, op by op as the reference's array ops evaluate
// it: 0.5*g*(1+tanh(c1*(g+c2*g^3)))*up, each op one fp32 operation.  In the bf16
// model dtype the qmm outputs, the constants (model_scalar) and every intermediate
// are bf16, so each op's result is rounded to bf16; under the float32 override all
// stay fp32.  Contraction is off: an FMA would skip the rounding of a product (hipcc
// contracts by default, also across the header's __fmul_rn / __fadd_rn, which are
// plain operators).  g^3 is g*g*g: exact in fp32 for a bf16 g (at most 24
// significant bits), and within an ulp of the reference's pow(g, 3) for an fp32 g.
// gelu of a bf16 g in the bf16 op sequence: a function of g's 16 bits only, so the
// GEMM epilogue reads it from a table built by this same code (see kGeluTable).
__device__ __forceinline__ float gelu_bf16(float g) {
#pragma clang fp contract(off)
    const float c_tanh = 0.796875f;           // bf16(0.7978845608028654)
    const float c_cubic = 0.044677734375f;    // bf16(0.044715)
    const float g3 = round_bf16(g * g * g);
    const float a = round_bf16(g + round_bf16(c_cubic * g3));
    const float t = round_bf16(tanhf(round_bf16(c_tanh * a)));
    return round_bf16(round_bf16(0.5f * g) * round_bf16(1.0f + t));
}

__device__ __forceinline__ float geglu_bf16(float gate, float up) {
#pragma clang fp contract(off)
    return round_bf16(gelu_bf16(round_bf16(gate)) * round_bf16(up));
}

// gelu_bf16 over all 65536 bf16 patterns needs a table only for biased exponents
// 118..128 (|g| in [2^-9, 4)): below, 1 + t rounds to 1 and gelu = bf16(0.5 g);
// above, 1 + t is 2 (g > 0: gelu = g) or 0 (g < 0: gelu = -0); +inf gives +inf,
// -inf and NaN give NaN.  (Checked against the op sequence for every pattern.)
constexpr int kGeluExpLo = 118;
constexpr int kGeluExps = 11;
constexpr int kGeluTable = 2 * kGeluExps * 128;  // entries [sign][exponent - 118][mantissa]

// bf16 pattern of table entry i
__host__ __device__ constexpr uint32_t gelu_table_pattern(int i) {
    return ((uint32_t)(i / (kGeluExps * 128)) << 15) | ((uint32_t)(kGeluExpLo + (i / 128) % kGeluExps) << 7) |
           (uint32_t)(i % 128);
}

// GeGLU from the table (kGeluTable bf16 values, e.g. staged in LDS) and the closed forms
__device__ __forceinline__ float geglu_bf16_table(const uint16_t* table, float gate, float up) {
#pragma clang fp contract(off)
    const uint32_t b = f32_to_bf16(gate);
    const float g = __uint_as_float(b << 16);
    const uint32_t e = (b >> 7) & 0xFFu, neg = b >> 15, man = b & 0x7Fu;
    const int idx = (int)((neg * kGeluExps + (e - kGeluExpLo)) * 128u + man);
    const bool in_table = e >= (uint32_t)kGeluExpLo && e < (uint32_t)(kGeluExpLo + kGeluExps);
    const float looked = __uint_as_float((uint32_t)table[in_table ? idx : 0] << 16);
    float gelu;
    if (in_table)
        gelu = looked;
    else if (e < (uint32_t)kGeluExpLo)
        gelu = round_bf16(0.5f * g);
    else if (e < 255u)
        gelu = neg ? -0.0f : g;
    else
        gelu = (man == 0 && !neg) ? g : __uint_as_float(0xFFC00000u);
    return round_bf16(gelu * round_bf16(up));
}

__device__ __forceinline__ float geglu_f32(float g, float u) {
#pragma clang fp contract(off)
    const float c_tanh = 0.7978845608028654f, c_cubic = 0.044715f;
    const float g3 = g * g * g;
    const float a = g + c_cubic * g3;
    const float t = tanhf(c_tanh * a);
    const float gelu = (0.5f * g) * (1.0f + t);
    return gelu * u;
}

// The value of lane (l ^ 8) within each 16-lane row (DPP row_ror:8).  Every lane of
// the wave must execute it.
__device__ __forceinline__ float row_swap8(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
}

// The lm_head's final-logit softcap, tanh(logits / cap) * cap (native_model.cc:1794),
// op by op: bf16 rounding after the qmm output and after every op in the bf16 model
// dtype (cap is then bf16), all fp32 under the float32 override.  Division is IEEE
// (correctly rounded).  cap = 0 leaves the (rounded) logits as they are.
__device__ __forceinline__ float softcap_bf16(float v, float cap) {
#pragma clang fp contract(off)
    const float l = round_bf16(v);
    if (cap == 0.0f) return l;
    const float c = round_bf16(cap);
    return round_bf16(round_bf16(tanhf(round_bf16(l / c))) * c);
}
__device__ __forceinline__ float softcap_f32(float v, float cap) {
#pragma clang fp contract(off)
    return cap == 0.0f ? v : tanhf(v / cap) * cap;
}

// Greedy key of (value, index): unsigned order = value order, and on equal values the
// lower index is larger (argmax returns the first maximum).  0 is below every key.
__device__ __forceinline__ unsigned long long greedy_key(float v, int n) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (0xFFFFFFFFu - (uint32_t)n);
}
__device__ __forceinline__ float greedy_value(unsigned long long key) {
    const uint32_t o = (uint32_t)(key >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ int greedy_index(unsigned long long key) {
    return (int)(0xFFFFFFFFu - (uint32_t)key);
}

// Writes accumulator v of output row m, column 16*rb + col.  All lanes of the wave
// call it together (the GeGLU modes read the partner column from lane col ^ 8, the
// greedy modes reduce over the block's 16 columns); n_rows bounds the projection's N.
// Kernels never launched in the greedy modes compile that branch out (kGreedy).
template <bool kGreedy = true>
__device__ __forceinline__ void store_out(const OutParams& op, int m, int m_rows, int rb, int col, int n_rows,
                                          float v) {
    void* y = op.y;
    const int mode = op.mode;
    const int n_out = op.n_out;
    if (kGreedy && mode >= kOutGreedyBf16) {
        const int n = rb * 16 + col;
        const bool bf = mode == kOutGreedyBf16;
        const float c = bf ? softcap_bf16(v, op.cap) : softcap_f32(v, op.cap);
        const bool valid = m < m_rows && n < n_rows;
        if (valid && y != nullptr) {
            const long o = (long)m * n_rows + n;
            if (bf)
                static_cast<uint16_t*>(y)[o] = f32_to_bf16(c);
            else
                static_cast<float*>(y)[o] = c;
        }
        unsigned long long key = n < n_rows ? greedy_key(c, n) : 0ull;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {  // max over the 16 columns of this row
            const unsigned long long o = __shfl_xor(key, d);
            key = o > key ? o : key;
        }
        if (col == 0 && m < m_rows) op.part[(long)m * op.nb + rb] = key;
        return;
    }
    if (mode < kOutGegluBf16) {
        const int n = rb * 16 + col;
        if (m < m_rows && n < n_rows) {
            const long o = (long)m * n_rows + n;
            if (mode == kOutF32)
                static_cast<float*>(y)[o] = v;
            else
                static_cast<uint16_t*>(y)[o] = f32_to_bf16(v);
        }
    } else {
        const float up = row_swap8(v);
        const int hn = rb * 8 + col;
        if (col < 8 && m < m_rows && hn < n_out) {
            const long o = (long)m * n_out + hn;
            if (mode == kOutGegluF32)
                static_cast<float*>(y)[o] = geglu_f32(v, up);
            else
                static_cast<uint16_t*>(y)[o] = f32_to_bf16(geglu_bf16(v, up));
        }
    }
}

// GeGLU of two accumulators of one column, rows m0 (v0) and m1 (v1), with every lane
// doing useful work: lanes col < 8 hold gate, lanes col >= 8 up.  After one exchange
// lane col < 8 has (gate, up) of row m0 for h column 8*rb + col, and lane col >= 8
// has (gate, up) of row m1 for h column 8*rb + col - 8 (geglu2_row / geglu2_col give
// the lane's output coordinates).  All lanes of the wave call it together.  In bf16
// gelu comes from `table` (gelu_bf16 of every bf16 pattern).
__device__ __forceinline__ float geglu2(int mode, int col, float v0, float v1, const uint16_t* __restrict__ table) {
    const bool lo = col < 8;
    const float other = row_swap8(lo ? v1 : v0);  // lo: up of row m0; hi: gate of row m1
    const float g = lo ? v0 : other;
    const float u = lo ? other : v1;
    return mode == kOutGegluF32 ? geglu_f32(g, u) : geglu_bf16_table(table, g, u);
}
__device__ __forceinline__ int geglu2_row(int col, int m0, int m1) { return col < 8 ? m0 : m1; }
__device__ __forceinline__ int geglu2_col(int col, int rb) { return rb * 8 + (col & 7); }

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// LDS DMA (buffer_load ... lds) issued from asm, and explicit vmcnt waits
// ---------------------------------------------------------------------------
// 16-byte-per-lane DMA into LDS: lane i's 16 bytes land at lds + 16 i, read from
// voff + soff.  Only voff is checked against the buffer's size (a resource of size
// 0 reads zeros for any offset); callers keep voff + soff inside the buffer for
// in-range lanes and put the rest at kOutOfRange.  Issued as
// inline asm, so the compiler does not track it: it would otherwise insert waits for
// all outstanding DMAs before LDS reads it cannot tell apart from them (it keeps at
// most eight DMA records), undoing the prefetch.  Ordering is this kernel's own: every
// DMA'd slot is read only after an explicit vmcnt wait and a barrier.  M0 (the LDS
// address) is an operand, so the compiler knows it is written.  The compiler's hazard
// checks cannot see into the asm, so it opens with the wait states the load may need:
// 5 after a VALU write of an SGPR it reads (under register pressure the compiler
// reloads resource and offset SGPRs from VGPR lanes with v_readlane right before it),
// which also covers the 1 an M0 write needs.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, const void* lds, uint32_t voff, uint32_t soff = 0) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);  // LDS offset: low half of the generic address
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(m0)
                 : "memory");
}

// s_waitcnt with vmcnt(n) only (expcnt / lgkmcnt left free), n < 64
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");  // the builtin is not a memory operation: keep loads after it
}
// the same plus lgkmcnt(0): this wave's LDS reads have returned
template <int N>
__device__ __forceinline__ void wait_vm_lds() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}

// lgkmcnt(0) only: this wave's LDS reads have returned
__device__ __forceinline__ void wait_lds() {
    __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
    asm volatile("" ::: "memory");
}

// s_barrier without __syncthreads' fence (which would wait for every outstanding
// load); the empty asm keeps LDS accesses on their side of it for the compiler
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

}  // namespace q4
