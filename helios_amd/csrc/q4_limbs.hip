// Decode-shape affine-Q4 matmul on the int8 matrix cores (gfx950), for one row of x.
//
// The weight side needs no conversion beyond a mask: with the tiled words of the
// record layout (q4_common.h), `word & 0x78787878` puts four nibbles in bits 3..6 of
// four bytes, i.e. the int8 values 8q, and `rotr(word, 4) & 0x78787878` the other four.
// So the 16 nibbles a lane holds for one group become the 16 int8 B operands of one
// v_mfma_i32_16x16x64_i8 with three VALU ops per word (the bf16 kernels need seven
// per word for 1 + q/16, and two 16x16x32 MFMAs per group instead of one).
//
// The x side is split exactly into int8 limbs, once per workgroup.  For group g with
// largest |x| below 2^(e-126) (e the biased exponent), V = rint(x * 2^(146-e)) is an
// integer with |V| < 2^20 (x * 2^(132-e) is below 64 in magnitude), and
//     V = 16384 * L0 + 128 * L1 + L2,   L0 = V >> 14 in [-64, 63], L1, L2 in [0, 127].
// Every x whose exponent is within 12 of the group maximum is exact in this form; the
// rest are rounded at 2^-21 of the group maximum, below the fp32 rounding of a
// 64-term sum of products.  The matrix cores then form exact int32 sums
//     C_l = sum_k L_l(x_k) * 8 q_k,
// and  sum_k x_k q_k = (C0 + C1 / 128 + C2 / 16384) * 2^(e-135)  in fp32.  With the
// group's scale s and bias b:  y += s * sum(x q) + b * X_g  (X_g the fp32 group sum,
// kept in units of 2^(e-132); s and b take the power of two before the products, so
// an intermediate overflows only where y does).
//
// Four groups share one accumulator: the MFMA of group 4c + j reads A rows 4j + l
// (limb l < 3 of x on that group's 64 columns, zero elsewhere), so after the four
// MFMAs of a chunk, lane (quarter j, column n) holds C_0..C_2 of group 4c + j for
// output column n in its first three accumulator registers, and every lane's scale
// step is useful work (10 VALU ops per chunk of four groups).
//
// Work split: a workgroup owns a contiguous range of whole 16-row blocks, whose
// records are one contiguous run of memory; its waves split that run's chunks (two
// records, four groups) evenly, each streaming its own contiguous part with NBUF
// chunks in flight.  A wave stores the row blocks it covers whole; the blocks shared
// by several waves are summed after one barrier, in wave order, by the first wave
// that touches them (deterministic: the same order on every run).
#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kByteNibMask = 0x78787878u;  // bits 3..6 of each byte: the int8 value 8q
constexpr int kLimbUnitBytes = 16;              // one lane's 16 int8 A operands
// LDS per chunk of four groups: [group j][limb l][k-quarter] units, then one zero unit
// read by every lane whose A row is zero in that MFMA
constexpr int kLimbChunkBytes = 4 * 3 * 4 * kLimbUnitBytes;  // 768
constexpr int kLimbChunkStride = kLimbChunkBytes + kLimbUnitBytes;

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kNonTemporal);
}

// int8 B operands of one group from the lane's two words (half 0, half 1): bytes of
// value 8q in the order nibble (0, 4, 1, 5), (2, 6, 3, 7) of each word
__device__ __forceinline__ i32x4 expand_i8(uint32_t w0, uint32_t w1) {
    i32x4 b;
    b[0] = (int32_t)(w0 & kByteNibMask);
    b[1] = (int32_t)(rotr(w0, 4) & kByteNibMask);
    b[2] = (int32_t)(w1 & kByteNibMask);
    b[3] = (int32_t)(rotr(w1, 4) & kByteNibMask);
    return b;
}

// Byte 0 of a, b, c, d as one dword (a lowest).
__device__ __forceinline__ uint32_t pack_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0C0C0400u);  // a.b0, b.b0
    const uint32_t hi = __builtin_amdgcn_perm(d, c, 0x04000C0Cu);  // c.b0, d.b0 in bytes 2, 3
    return lo | hi;
}

template <int NBUF, int WAVES, bool STRIDED>
__global__ __launch_bounds__(WAVES * 64) void decode_limb_kernel(const uint4* __restrict__ tiles,
                                                                 const uint16_t* __restrict__ x, OutParams op,
                                                                 int n_rows, int k, int kx, int gpairs, int nblocks) {
    extern __shared__ uint4 lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int quarter = lane >> 4;
    const int groups = k >> 6;
    const int nch = (gpairs + 1) >> 1;  // chunks of two records per row block
    // the workgroup's row blocks: rb0 + i * rbs, i < nrb (STRIDED: every gridDim.x-th
    // block, so that the grid's requests at any time lie in one region; else a
    // contiguous range)
    const int rb0 = STRIDED ? (int)blockIdx.x : (int)(((uint32_t)blockIdx.x * (uint32_t)nblocks) / gridDim.x);
    const int nrb = STRIDED ? (nblocks - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x
                            : (int)(((uint32_t)blockIdx.x * (uint32_t)nblocks + (uint32_t)nblocks) / gridDim.x) - rb0;
    const int rbs = STRIDED ? (int)gridDim.x : 1;
    const int total = nrb * nch;  // chunks of the workgroup's run, block-major
    char* const limbs = reinterpret_cast<char*>(lds);
    float2* const tab = reinterpret_cast<float2*>(limbs + nch * kLimbChunkStride);  // [nch * 4] (2^(e-135), X_g)
    float* const slots = reinterpret_cast<float*>(tab + nch * 4);                   // [nrb][WAVES][16]

    // lane (quarter j, column n) holds group 4c + j's scale word for row n: record j / 2
    // of the chunk, word j % 2
    const uint32_t sb_off = (uint32_t)((quarter >> 1) * kRecBytes + kRecSbBytes + col * 8 + (quarter & 1) * 4);

    uint4 t0[NBUF], t1[NBUF];
    uint32_t sw[NBUF];
    // Wave w takes chunks w, w + WAVES, ... of the run, so the workgroup's requests in
    // flight cover one contiguous window of the records.  Issue cursor: flat chunk and
    // its (row block, chunk) within the run.
    int i_f = wave, i_rb = 0, i_c = wave;
    while (i_c >= nch) {
        i_c -= nch;
        ++i_rb;
    }
    // Chunks past the run read an empty range (zeros, no traffic): every loop iteration
    // issues the same loads, which keeps the compiler's wait counts exact.
    auto issue = [&](int b) {
        const bool live = i_f < total;
        const int left = gpairs - 2 * i_c;
        const int nrec = !live ? 0 : left < 2 ? left : 2;
        const long first = live ? (long)(rb0 + i_rb * rbs) * gpairs + 2 * i_c : 0;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(tiles + first * kRecU4, (uint32_t)nrec * kRecBytes);
        t0[b] = buffer_load16<kNonTemporal>(rs, (uint32_t)(lane * 16));
        t1[b] = buffer_load16<kNonTemporal>(rs, (uint32_t)(kRecBytes + lane * 16));
        sw[b] = buffer_load4(rs, sb_off);
        i_f += WAVES;
        i_c += WAVES;
        while (i_c >= nch) {
            i_c -= nch;
            ++i_rb;
        }
    };

    // x' -> int8 limbs in LDS and (2^(e-135), X_g) per group.  Unit u is the 16-byte
    // unit u of the x' row: group u / 8, half (u / 4) % 2, k-quarter u % 4; the eight
    // units of a group are eight consecutive lanes.  Every thread runs every pass (the
    // group reductions are shuffles); units >= `units` are computed and dropped.
    constexpr int nthr = WAVES * 64;
    const int units = nch * 32;
    const int xunits = groups * 8;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)kx * 2u);
    auto load_unit = [&](int u) { return buffer_load16(xrs, u < xunits ? xprime_offset(u, k, kx) : kOutOfRange); };
    auto stage = [&](const uint4 v, int u) {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
        // group maximum of |x| as bf16 magnitude bits (integer order = value order; inf
        // and NaN sort above every finite value)
        uint32_t mb = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = w4[j] & 0x7FFFu, hi = (w4[j] >> 16) & 0x7FFFu;
            mb = mb > lo ? mb : lo;
            mb = mb > hi ? mb : hi;
        }
        mb = octet_max(mb);
        const int ex = (int)(mb >> 7);  // biased exponent of the group maximum
        const int e = ex < 19 ? 19 : ex > 254 ? 254 : ex;
        const float scale = __uint_as_float((uint32_t)(273 - e) << 23);   // 2^(146 - e)
        const float unit = __uint_as_float((uint32_t)(259 - e) << 23);    // 2^(132 - e)
        // the group sum in units of 2^(e-132), |x| * 2^(132-e) < 64 (so no sum of x
        // near the largest finite values overflows)
        float sum = 0.f;
        uint32_t l0[8], l1[8], l2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xv = (i & 1) ? bf16_hi(w4[i >> 1]) : bf16_lo(w4[i >> 1]);
            sum += xv * unit;
            // x * 2^(146-e) + 1.5 * 2^23 (one rounding, to nearest even): the low 22 bits
            // of the result are V in two's complement
            const uint32_t bits = __float_as_uint(__builtin_fmaf(xv, scale, 12582912.0f));
            l2[i] = bits;                                               // V & 127 after the mask
            l1[i] = bits >> 7;                                          // (V >> 7) & 127 after the mask
            l0[i] = (uint32_t)__builtin_amdgcn_sbfe((int)bits, 14, 8);  // V >> 14
        }
        sum = octet_sum(sum);
        // slot order within a half: nibbles (0, 4, 1, 5), (2, 6, 3, 7)
        const uint2 p0 = make_uint2(pack_bytes(l0[0], l0[4], l0[1], l0[5]), pack_bytes(l0[2], l0[6], l0[3], l0[7]));
        const uint2 p1 = make_uint2(pack_bytes(l1[0], l1[4], l1[1], l1[5]) & 0x7F7F7F7Fu,
                                    pack_bytes(l1[2], l1[6], l1[3], l1[7]) & 0x7F7F7F7Fu);
        const uint2 p2 = make_uint2(pack_bytes(l2[0], l2[4], l2[1], l2[5]) & 0x7F7F7F7Fu,
                                    pack_bytes(l2[2], l2[6], l2[3], l2[7]) & 0x7F7F7F7Fu);
        if (u < units) {
            const int g = u >> 3, h = (u >> 2) & 1, kq = u & 3;
            char* const base = limbs + (g >> 2) * kLimbChunkStride + (g & 3) * 192 + kq * 16 + h * 8;
            *reinterpret_cast<uint2*>(base) = p0;
            *reinterpret_cast<uint2*>(base + 64) = p1;
            *reinterpret_cast<uint2*>(base + 128) = p2;
            if ((u & 7) == 0) {
                // 2^(e-135) (NaN for a group holding inf or NaN, so that it reaches y) and
                // 8 X_g 2^(132-e)
                const float fs = ex == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float((uint32_t)(e - 8) << 23);
                tab[g] = make_float2(fs, 8.0f * sum);
            }
        }
    };
    // the first two passes of x are requested before the weights (loads complete in
    // order: waiting for an x load issued after them would wait for every weight load)
    const uint4 xa = load_unit((int)threadIdx.x);
    const uint4 xb = load_unit(nthr + (int)threadIdx.x);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) issue(b);
    stage(xa, (int)threadIdx.x);
    if (nthr < units) stage(xb, nthr + (int)threadIdx.x);
    for (int u0 = 2 * nthr; u0 < units; u0 += nthr) stage(load_unit(u0 + (int)threadIdx.x), u0 + (int)threadIdx.x);
    for (int c = (int)threadIdx.x; c < nch; c += nthr)
        *reinterpret_cast<uint4*>(limbs + c * kLimbChunkStride + kLimbChunkBytes) = make_uint4(0, 0, 0, 0);
    // (row block, wave) slots a wave never writes stay zero
    for (int t = (int)threadIdx.x; t < nrb * WAVES * 16; t += nthr) slots[t] = 0.f;
    __syncthreads();

    // A operand address of MFMA j within a chunk: lane (row r = col, k-quarter) reads
    // limb r % 4 of group j when r / 4 == j and r % 4 < 3, else the zero unit
    uint32_t a_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        a_off[j] = ((col >> 2) == j && (col & 3) < 3) ? (uint32_t)(j * 192 + (col & 3) * 64 + quarter * 16)
                                                      : (uint32_t)kLimbChunkBytes;

    float acc = 0.f;
    int c_f = wave, c_rb = 0, c_c = wave;  // compute cursor
    while (c_c >= nch) {
        c_c -= nch;
        ++c_rb;
    }
    auto compute = [&](int b) {
        const char* const cl = limbs + c_c * kLimbChunkStride;
        i32x4 C = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 t = (j >> 1) ? t1[b] : t0[b];
            const i32x4 B = (j & 1) ? expand_i8(t.z, t.w) : expand_i8(t.x, t.y);
            const i32x4 A = *reinterpret_cast<const i32x4*>(cl + a_off[j]);
            C = mfma_i8(A, B, C);
        }
        // y += s * sum(x q) + b * X_g = (s 2^(e-135)) P + (b 2^(e-135)) (8 X_g 2^(132-e));
        // the scale and bias take the power of two first, so that no intermediate
        // overflows where y itself does not
        const float2 tv = tab[c_c * 4 + quarter];
        const float p = __builtin_fmaf(__builtin_fmaf((float)C[2], 0x1p-7f, (float)C[1]), 0x1p-7f, (float)C[0]);
        acc = __builtin_fmaf(bf16_lo(sw[b]) * tv.x, p, acc);
        acc = __builtin_fmaf(bf16_hi(sw[b]) * tv.x, tv.y, acc);
        // advance; the sum leaves for the block's slot when the wave's next chunk lies
        // in another row block (or there is none)
        const int rb = c_rb;
        c_f += WAVES;
        c_c += WAVES;
        while (c_c >= nch) {
            c_c -= nch;
            ++c_rb;
        }
        if (c_rb != rb || c_f >= total) {
            float v = acc + __shfl_xor(acc, 16);
            v += __shfl_xor(v, 32);
            if (quarter == 0) slots[(rb * WAVES + wave) * 16 + col] = v;
            acc = 0.f;
        }
    };

    const int mine = wave < total ? (total - wave + WAVES - 1) / WAVES : 0;  // chunks of this wave
    int i = 0;
    for (; i + NBUF <= mine; i += NBUF) {
#pragma unroll
        for (int b = 0; b < NBUF; ++b) {
            compute(b);
            issue(b);
        }
    }
#pragma unroll
    for (int b = 0; b + 1 < NBUF; ++b)
        if (i + b < mine) compute(b);

    __syncthreads();
    // every row block's 16 outputs: the waves' slots summed in wave order; a 16-lane
    // row of a wave holds one block (the GeGLU and greedy stages work within it)
    for (int t0 = 0; t0 < nrb * 16; t0 += nthr) {
        const int t = t0 + (int)threadIdx.x;
        const int r = t >> 4;
        float v = 0.f;
        if (t < nrb * 16) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) v += slots[(r * WAVES + w) * 16 + col];
        }
        store_out(op, t < nrb * 16 ? 0 : 1, 1, rb0 + r * rbs, col, n_rows, v);
    }
}

// Rows 2-8 of x (MT = 2, 4 or 8, the rows padded with zeros) on the int8 matrix cores,
// the same limb split per (row, group).  The A rows of one MFMA are (group, row, limb)
// triples with a zero row after each (row, group)'s three limbs:
//   MT <= 4: the MFMA of group j of a chunk feeds accumulator j / (4 / MT); within it
//            rows 4 MT (j % (4 / MT)) + 4m + l hold limb l of row m, so lane
//            (quarter q, column n) ends with C_0..C_2 of group (q / MT) of that
//            accumulator and row q % MT;
//   MT = 8:  two MFMAs per group j on the same B operand, accumulators 2j and 2j + 1,
//            rows 4m' + l of row 4h + m' (h = 0, 1), so lane (q, n) holds row 4h + q.
// A lane accumulates one row (MT <= 4) or two (MT = 8); its scale words are those of
// the groups it holds, two 4- or 8-byte loads per chunk.  Per chunk: 4 MFMAs (8 at
// MT = 8) and MT scale steps per lane.
// BATCH = 0: the per-(row block, wave) sums of the whole run stay in LDS to the end.
// BATCH > 0 (long runs, one workgroup per CU that stages x once): the run goes in
// phases of BATCH row blocks whose sums take one half of a two-phase ring; at each
// phase's end the waves meet at a barrier and sum (in wave order) and store that
// phase's outputs, clearing its half for the phase after next, while the next phase's
// loads stay in flight.
template <int MT, int NBUF, int WAVES, bool STRIDED, int BATCH = 0>
__global__ __launch_bounds__(WAVES * 64) void decode_limb_rows_kernel(const uint4* __restrict__ tiles,
                                                                      const uint16_t* __restrict__ x, OutParams op,
                                                                      int m_rows, int n_rows, int k, int kx,
                                                                      int gpairs, int nblocks) {
    static_assert(MT == 2 || MT == 4 || MT == 8, "rows");
    constexpr int kGpa = MT <= 4 ? 4 / MT : 1;  // groups per accumulator
    constexpr int kAcc = MT;                     // accumulators per chunk
    constexpr int kMfma = MT <= 4 ? 4 : 8;       // MFMAs per chunk
    constexpr int kRows = MT <= 4 ? 1 : 2;       // rows a lane accumulates
    constexpr int kChunkBytes = 4 * MT * 3 * kLimbUnitBytes * 4;  // [group][row][limb][quarter] x 16 B
    constexpr int kChunkStride = kChunkBytes + kLimbUnitBytes;    // then one zero unit
    extern __shared__ uint4 lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int quarter = lane >> 4;
    const int groups = k >> 6;
    const int nch = (gpairs + 1) >> 1;
    const int rb0 = STRIDED ? (int)blockIdx.x : (int)(((uint32_t)blockIdx.x * (uint32_t)nblocks) / gridDim.x);
    const int nrb = STRIDED ? (nblocks - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x
                            : (int)(((uint32_t)blockIdx.x * (uint32_t)nblocks + (uint32_t)nblocks) / gridDim.x) - rb0;
    const int rbs = STRIDED ? (int)gridDim.x : 1;
    const int total = nrb * nch;
    char* const limbs = reinterpret_cast<char*>(lds);
    float2* const tab = reinterpret_cast<float2*>(limbs + nch * kChunkStride);  // [nch][4][MT] (2^(e-135), 8 X 2^(132-e))
    // [nrb][WAVES][MT][16], or with BATCH the ring [2][BATCH][WAVES][MT][16]
    float* const slots = reinterpret_cast<float*>(tab + nch * 4 * MT);
    const int slot_rbs = BATCH ? 2 * BATCH : nrb;

    // scale words: MT = 2: groups q/2 (record 0) and 2 + q/2 (record 1), 4 bytes each;
    // MT >= 4: all four groups, 8 bytes of each record
    const uint32_t sb0 = (uint32_t)(kRecSbBytes + col * 8 + (MT == 2 ? (quarter >> 1) * 4 : 0));
    uint4 t0[NBUF], t1[NBUF];
    uint32_t sw[NBUF][4];
    int i_f = wave, i_rb = 0, i_c = wave;
    while (i_c >= nch) {
        i_c -= nch;
        ++i_rb;
    }
    auto issue = [&](int b) {
        const bool live = i_f < total;
        const int left = gpairs - 2 * i_c;
        const int nrec = !live ? 0 : left < 2 ? left : 2;
        const long first = live ? (long)(rb0 + i_rb * rbs) * gpairs + 2 * i_c : 0;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(tiles + first * kRecU4, (uint32_t)nrec * kRecBytes);
        t0[b] = buffer_load16<kNonTemporal>(rs, (uint32_t)(lane * 16));
        t1[b] = buffer_load16<kNonTemporal>(rs, (uint32_t)(kRecBytes + lane * 16));
        if constexpr (MT == 2) {
            sw[b][0] = buffer_load4(rs, sb0);
            sw[b][1] = buffer_load4(rs, kRecBytes + sb0);
        } else {
            const uint2 a = buffer_load8<kNonTemporal>(rs, sb0);
            const uint2 c = buffer_load8<kNonTemporal>(rs, kRecBytes + sb0);
            sw[b][0] = a.x;
            sw[b][1] = a.y;
            sw[b][2] = c.x;
            sw[b][3] = c.y;
        }
        i_f += WAVES;
        i_c += WAVES;
        while (i_c >= nch) {
            i_c -= nch;
            ++i_rb;
        }
    };

    // x' rows -> limbs; unit f = m * (nch * 32) + u, u the 16-byte unit of row m's x'
    // (group u / 8, half (u / 4) % 2, k-quarter u % 4): the eight units of a (row,
    // group) are eight consecutive lanes.  Rows >= m_rows and groups past K stage zeros.
    constexpr int nthr = WAVES * 64;
    const int runits = nch * 32;
    const int units = MT * runits;
    const int xunits = groups * 8;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)kx * 2u);
    auto load_unit = [&](int f) {
        const int m = f / runits, u = f - m * runits;
        const bool ok = m < m_rows && u < xunits;
        return buffer_load16(xrs, ok ? (uint32_t)m * (uint32_t)kx * 2u + xprime_offset(u, k, kx) : kOutOfRange);
    };
    auto stage = [&](const uint4 v, int f) {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
        uint32_t mb = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = w4[j] & 0x7FFFu, hi = (w4[j] >> 16) & 0x7FFFu;
            mb = mb > lo ? mb : lo;
            mb = mb > hi ? mb : hi;
        }
        mb = octet_max(mb);
        const int ex = (int)(mb >> 7);
        const int e = ex < 19 ? 19 : ex > 254 ? 254 : ex;
        const float scale = __uint_as_float((uint32_t)(273 - e) << 23);  // 2^(146 - e)
        const float unit = __uint_as_float((uint32_t)(259 - e) << 23);   // 2^(132 - e)
        float sum = 0.f;
        uint32_t l0[8], l1[8], l2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xv = (i & 1) ? bf16_hi(w4[i >> 1]) : bf16_lo(w4[i >> 1]);
            sum += xv * unit;
            const uint32_t bits = __float_as_uint(__builtin_fmaf(xv, scale, 12582912.0f));
            l2[i] = bits;
            l1[i] = bits >> 7;
            l0[i] = (uint32_t)__builtin_amdgcn_sbfe((int)bits, 14, 8);
        }
        sum = octet_sum(sum);
        const uint2 p0 = make_uint2(pack_bytes(l0[0], l0[4], l0[1], l0[5]), pack_bytes(l0[2], l0[6], l0[3], l0[7]));
        const uint2 p1 = make_uint2(pack_bytes(l1[0], l1[4], l1[1], l1[5]) & 0x7F7F7F7Fu,
                                    pack_bytes(l1[2], l1[6], l1[3], l1[7]) & 0x7F7F7F7Fu);
        const uint2 p2 = make_uint2(pack_bytes(l2[0], l2[4], l2[1], l2[5]) & 0x7F7F7F7Fu,
                                    pack_bytes(l2[2], l2[6], l2[3], l2[7]) & 0x7F7F7F7Fu);
        if (f < units) {
            const int m = f / runits, u = f - m * runits;
            const int g = u >> 3, h = (u >> 2) & 1, kq = u & 3;
            char* const base = limbs + (g >> 2) * kChunkStride + (((g & 3) * MT + m) * 3) * 64 + kq * 16 + h * 8;
            *reinterpret_cast<uint2*>(base) = p0;
            *reinterpret_cast<uint2*>(base + 64) = p1;
            *reinterpret_cast<uint2*>(base + 128) = p2;
            if ((u & 7) == 0) {
                const float fs = ex == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float((uint32_t)(e - 8) << 23);
                tab[(g >> 2) * 4 * MT + (g & 3) * MT + m] = make_float2(fs, 8.0f * sum);
            }
        }
    };
    // the first kPre passes of x are requested before the weights (loads complete in
    // order: an x load issued after them waits for every weight load in flight); 8
    // rows of K = 3840-4096, and 2 rows of K = 15360 (the 16-wave launches of long K),
    // take four passes of 1024 threads.  (Four for the other launches cost their
    // registers: the pair at 2 rows 13.13 -> 13.46 us.)
    constexpr int kPre = MT == 8 || (MT == 2 && WAVES == 16) ? 4 : 2;
    uint4 xp[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) xp[i] = load_unit(i * nthr + (int)threadIdx.x);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) issue(b);
#pragma unroll
    for (int i = 0; i < kPre; ++i)
        if (i == 0 || i * nthr < units) stage(xp[i], i * nthr + (int)threadIdx.x);
    for (int f0 = kPre * nthr; f0 < units; f0 += nthr) stage(load_unit(f0 + (int)threadIdx.x), f0 + (int)threadIdx.x);
    for (int c = (int)threadIdx.x; c < nch; c += nthr)
        *reinterpret_cast<uint4*>(limbs + c * kChunkStride + kChunkBytes) = make_uint4(0, 0, 0, 0);
    for (int t = (int)threadIdx.x; t < slot_rbs * WAVES * MT * 16; t += nthr) slots[t] = 0.f;
    __syncthreads();

    // BATCH: the end of phase ph (row blocks [ph BATCH, ph BATCH + BATCH) of the run):
    // every wave's sums of it are in LDS after the barrier; each (row block, row)'s 16
    // outputs are the waves' slots summed in wave order (a 16-lane row holds one, as the
    // GeGLU and greedy stages need), and the slots read are cleared for phase ph + 2
    int phase = 0;
    auto end_phase = [&](int ph) {
        wait_lds();
        lds_barrier();
        const int r0 = ph * BATCH;
        const int half = (ph & 1) * BATCH;
        for (int t0 = 0; t0 < BATCH * MT * 16; t0 += nthr) {
            const int t = t0 + (int)threadIdx.x;
            const int r = t / (MT * 16), m = (t >> 4) % MT;
            const bool live = t < BATCH * MT * 16 && r0 + r < nrb;
            float v = 0.f;
            if (t < BATCH * MT * 16) {
#pragma unroll
                for (int w = 0; w < WAVES; ++w) {
                    float* const sl = slots + (((half + r) * WAVES + w) * MT + m) * 16 + col;
                    v += *sl;
                    *sl = 0.f;
                }
            }
            store_out(op, live ? m : MT, m_rows, rb0 + (live ? r0 + r : 0) * rbs, col, n_rows, v);
        }
    };
    (void)phase;
    (void)end_phase;

    // A operand address of MFMA i of a chunk for this lane (row r = col, k-quarter)
    uint32_t a_off[kMfma];
#pragma unroll
    for (int i = 0; i < kMfma; ++i) {
        const int r = col, l = r & 3;
        int j, m;
        bool on;
        if constexpr (MT <= 4) {
            j = i;
            m = (r % (4 * MT)) >> 2;
            on = (r / (4 * MT)) == (i % kGpa) && l < 3;
        } else {
            j = i >> 1;
            m = 4 * (i & 1) + (r >> 2);
            on = l < 3;
        }
        a_off[i] = on ? (uint32_t)(((j * MT + m) * 3 + l) * 64 + quarter * 16) : (uint32_t)kChunkBytes;
    }

    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = 0.f;
    int c_f = wave, c_rb = 0, c_c = wave;
    while (c_c >= nch) {
        c_c -= nch;
        ++c_rb;
    }
    auto compute = [&](int b) {
        if constexpr (BATCH > 0) {
            // the phases this wave's next chunk leaves behind end first
            while (phase < c_rb / BATCH) end_phase(phase++);
        }
        const char* const cl = limbs + c_c * kChunkStride;
        i32x4 C[kAcc];
#pragma unroll
        for (int a = 0; a < kAcc; ++a) C[a] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < kMfma; ++i) {
            const int j = MT <= 4 ? i : i >> 1;
            const int a = MT <= 4 ? i / kGpa : i;
            const uint4 t = (j >> 1) ? t1[b] : t0[b];
            const i32x4 B = (j & 1) ? expand_i8(t.z, t.w) : expand_i8(t.x, t.y);
            const i32x4 A = *reinterpret_cast<const i32x4*>(cl + a_off[i]);
            C[a] = mfma_i8(A, B, C[a]);
        }
        const float2* const tc = tab + c_c * 4 * MT;
#pragma unroll
        for (int a = 0; a < kAcc; ++a) {
            // the lane's (group, row) in accumulator a, and its scale word
            const int j = MT <= 4 ? a * kGpa + quarter / MT : a >> 1;
            const int m = MT <= 4 ? quarter % MT : 4 * (a & 1) + quarter;
            const uint32_t w = MT == 2 ? sw[b][a] : MT == 4 ? sw[b][a] : sw[b][a >> 1];
            const float2 tv = tc[j * MT + m];
            // C_1 128 + C_2 is exact in int32 (|C_1|, |C_2| < 64 * 127 * 120 < 2^20)
            const float p = __builtin_fmaf((float)(C[a][1] * 128 + C[a][2]), 0x1p-14f, (float)C[a][0]);
            float& r = acc[MT <= 4 ? 0 : (a & 1)];
            r = __builtin_fmaf(bf16_lo(w) * tv.x, p, r);
            r = __builtin_fmaf(bf16_hi(w) * tv.x, tv.y, r);
        }
        const int rb = c_rb;
        c_f += WAVES;
        c_c += WAVES;
        while (c_c >= nch) {
            c_c -= nch;
            ++c_rb;
        }
        if (c_rb != rb || c_f >= total) {
            const int srb = BATCH ? ((rb / (BATCH ? BATCH : 1)) & 1) * BATCH + rb % (BATCH ? BATCH : 1) : rb;
            float* const sl = slots + (srb * WAVES + wave) * MT * 16;
            if constexpr (MT == 2) {
                const float v = acc[0] + __shfl_xor(acc[0], 32);
                if (quarter < 2) sl[quarter * 16 + col] = v;
            } else if constexpr (MT == 4) {
                sl[quarter * 16 + col] = acc[0];
            } else {
                sl[quarter * 16 + col] = acc[0];
                sl[(4 + quarter) * 16 + col] = acc[1];
            }
#pragma unroll
            for (int r = 0; r < kRows; ++r) acc[r] = 0.f;
        }
    };

    const int mine = wave < total ? (total - wave + WAVES - 1) / WAVES : 0;
    int i = 0;
    for (; i + NBUF <= mine; i += NBUF) {
#pragma unroll
        for (int b = 0; b < NBUF; ++b) {
            compute(b);
            issue(b);
        }
    }
#pragma unroll
    for (int b = 0; b + 1 < NBUF; ++b)
        if (i + b < mine) compute(b);

    if constexpr (BATCH > 0) {
        const int phases = (nrb + BATCH - 1) / BATCH;
        while (phase < phases) end_phase(phase++);
        // the loads issued past the run (zeros, no traffic) land before the end
        __builtin_amdgcn_s_waitcnt(0);
        return;
    }
    __syncthreads();
    // every (row block, row)'s 16 outputs: the waves' slots summed in wave order; a
    // 16-lane row of a wave holds one (row block, row) (the GeGLU and greedy stages
    // work within it)
    for (int t0 = 0; t0 < nrb * MT * 16; t0 += nthr) {
        const int t = t0 + (int)threadIdx.x;
        const bool live = t < nrb * MT * 16;
        const int r = t / (MT * 16), m = (t >> 4) % MT;
        float v = 0.f;
        if (live) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) v += slots[((r * WAVES + w) * MT + m) * 16 + col];
        }
        store_out(op, live ? m : MT, m_rows, rb0 + (live ? r : 0) * rbs, col, n_rows, v);
    }
}

}  // namespace

namespace {
// Launch shape per weight shape, from a sweep of {waves per workgroup, workgroups per
// CU, chunks in flight, block order} at one row (MI355X, us per launch in graph
// replays of back-to-back launches; the bf16 kernels' time in brackets):
//  * K of at least 32 chunks with no more row blocks than CUs (down_proj 3840x15360):
//    16 waves, 3 chunks in flight: 8.4 (9.6); 8 waves 9.1-9.3;
//  * up to 4 row blocks per CU: 8 waves, one workgroup per CU, 2 chunks in flight,
//    contiguous runs: gate 15360x3840 7.5 (9.2-9.9), qkv 8192x3840 5.45 (6.3),
//    o 3840x4096 4.07 (4.95), k 2048x3840 3.65 (4.5);
//  * more: 8 waves, three workgroups per CU, one chunk in flight each, blocks dealt
//    round the grid: the gate|up pair 2x15360x3840 12.2 (13.5-14.4), the lm_head
//    262144x3840 84.7 (87.7-88.5).
// Everything in flight at once was slower everywhere (gate with four chunks per wave
// and 16 waves: 9.4), as were waves walking contiguous sub-ranges of a workgroup's
// run instead of taking its chunks in turn (gate 12.0).
struct LimbConfig {
    int waves;     // per workgroup
    int per_cu;    // workgroups per CU
    int nbuf;      // chunks in flight per wave
    bool strided;  // workgroup b takes row blocks b, b + grid, ... (else a contiguous range)
};
LimbConfig limb_config(const Layout& l) {
    const int cus = device_cus();
    const int nch = (l.gp + 1) / 2;
    if (nch >= 32 && l.nb <= cus) return {16, 1, 3, false};
    if (l.nb <= 4 * cus) return {8, 1, 2, false};
    return {8, 3, 1, true};
}
int limb_grid(const Layout& l, const LimbConfig& c) {
    const int cap = device_cus() * c.per_cu;
    return l.nb < cap ? l.nb : cap;
}
}  // namespace

size_t limb_lds_bytes(const Layout& l) {
    const LimbConfig c = limb_config(l);
    const size_t nch = (size_t)(l.gp + 1) / 2;
    const int grid = limb_grid(l, c);
    const size_t nrb = ((size_t)l.nb + grid - 1) / grid;
    return nch * kLimbChunkStride + nch * 4 * sizeof(float2) + nrb * c.waves * 16 * sizeof(float);
}

namespace {
// Rows 2-8.  Launch shapes from a sweep at 4 and 8 rows (us per launch, graph replays
// of back-to-back launches; the bf16 kernels in brackets), 16-wave workgroups for the
// padded rows' longer scale steps:
//  * up to four row blocks per CU: one workgroup per CU, two chunks in flight,
//    contiguous runs: gate 15360x3840 9.5 / 11.6 (12.3 / 13.5);
//  * more, up to 16 per CU: two workgroups per CU, one chunk in flight, blocks dealt
//    round the grid: the gate|up pair 14.6 / 18.4 (19.1 / 20.4); at 8 rows the LDS
//    admits one workgroup per CU and two chunks are in flight (16.3-16.7 against
//    16.7-17.2 us with one, x's passes all requested first);
//  * more still (the lm_head): one 16-wave workgroup per CU, two chunks in flight,
//    blocks dealt round the grid, the run walked in phases of two row blocks (the
//    kernel's BATCH): 90.3-91.2 / 102-104.6 (98.2 / 114-119.5);
// At 2 rows the one-row kernel's shapes.  Workgroups per CU are capped by what LDS
// admits (the per-(row block, wave) sums take MT times the one-row kernel's room), and
// the grid grows (more, shorter row-block runs) until one workgroup fits.
struct LimbRowsPlan {
    LimbConfig c;
    int grid;
    size_t lds;
    int batch = 0;  // row blocks per phase (the kernel's BATCH), 0: none
};
constexpr int kLimbBatch = 2;
size_t limb_rows_lds(const Layout& l, int mt, int waves, int grid, int batch = 0) {
    const size_t nch = (size_t)(l.gp + 1) / 2;
    const size_t nrb = batch ? 2 * (size_t)batch : ((size_t)l.nb + grid - 1) / grid;
    return nch * ((size_t)4 * mt * 3 * 64 + kLimbUnitBytes) + nch * 4 * mt * sizeof(float2) +
           nrb * waves * mt * 16 * sizeof(float);
}
LimbRowsPlan limb_rows_plan(const Layout& l, int mt) {
    LimbRowsPlan p;
    const int cus = device_cus();
    if (mt >= 4 && l.nb > 16 * cus) {
        // the lm_head: one 16-wave workgroup per CU stages x once and walks its run in
        // phases of two row blocks (4 / 8 rows: 91.2 / 104.6 us against 98.2 / 122.2 with
        // a workgroup per few row blocks, each staging x; 8 waves and phases of 4 or 8
        // row blocks, or 3 chunks in flight: 1-3% slower at 8 rows)
        p.c = {16, 1, 2, true};
        p.batch = kLimbBatch;
        p.grid = cus;
        p.lds = limb_rows_lds(l, mt, p.c.waves, p.grid, p.batch);
        if (p.lds <= (size_t)160 * 1024) return p;
        p.batch = 0;
    }
    if (mt == 2)
        p.c = limb_config(l);
    else if (l.nb <= 4 * cus)
        p.c = {16, 1, 2, false};
    else if (l.nb <= 16 * cus)
        p.c = {16, 2, mt == 8 ? 2 : 1, true};
    else
        p.c = {8, 2, 2, true};
    int per_cu = p.c.per_cu;
    for (;;) {
        p.grid = l.nb < cus * per_cu ? l.nb : cus * per_cu;
        p.lds = limb_rows_lds(l, mt, p.c.waves, p.grid);
        const int fit = (int)(((size_t)160 * 1024) / p.lds);
        if (fit >= per_cu || per_cu == 1) break;
        per_cu = fit > 1 ? fit : 1;
    }
    while (p.lds > (size_t)160 * 1024 && p.grid < l.nb) {
        p.grid = p.grid * 2 < l.nb ? p.grid * 2 : l.nb;
        p.lds = limb_rows_lds(l, mt, p.c.waves, p.grid);
    }
    return p;
}
int rows_mt(int m) { return m <= 2 ? 2 : m <= 4 ? 4 : 8; }
}  // namespace

size_t limb_rows_lds_bytes(const Layout& l, int m) { return limb_rows_plan(l, rows_mt(m)).lds; }

bool limb_rows_preferred(const Layout& l, int m) {
    if (m == 2) return true;
    // 3-8 rows: wide 4-bit outputs gain (the lm_head at 8 rows 102-104.6 us phased
    // against 114 for the bf16 kernels); narrower ones at 4 rows with K up to 4096 (qkv
    // 8192x3840 6.8 against 7.3 us, o 3840x4096 5.2 against 5.4, q 5.2 against 5.4, k
    // 2048x3840 4.9 against 5.0; 1024-wide K even; o of K = 8192 8.3 against 7.8) and
    // at 3 rows from 512 row blocks (qkv 6.8 against 7.1; q 5.3 against 5.2).  From 5
    // rows those lose (qkv 8.2 against 7.6-7.9 us, o 6.9 against 5.7).  The two-plane
    // 8-bit handles were not measured on these shapes.
    if (l.kx != l.k) return false;
    const int cus = device_cus();
    if (l.nb >= 3 * cus) return true;
    return l.gp <= 32 && ((m == 4 && l.nb >= 128) || (m == 3 && l.nb >= 2 * cus));
}

hipError_t launch_decode_limb_rows(const uint4* tiles, const uint16_t* x, const OutParams& op, int m,
                                   const Layout& l, hipStream_t stream) {
    const int mt = rows_mt(m);
    const LimbRowsPlan p = limb_rows_plan(l, mt);
    if (m < 2 || m > 8 || p.lds > (size_t)160 * 1024) return hipErrorInvalidValue;
    const dim3 grid(p.grid), block(64 * p.c.waves);
#define Q4_LR(MT, NB, W, ST)                                                                                     \
    hipLaunchKernelGGL((decode_limb_rows_kernel<MT, NB, W, ST>), grid, block, p.lds, stream, tiles, x, op, m, l.n, \
                       l.k, l.kx, l.gp, l.nb)
    if (mt == 2) {
        if (p.c.waves == 16)
            Q4_LR(2, 3, 16, false);
        else if (!p.c.strided)
            Q4_LR(2, 2, 8, false);
        else
            Q4_LR(2, 1, 8, true);
    } else if (p.batch) {
        if (mt == 4)
            hipLaunchKernelGGL((decode_limb_rows_kernel<4, 2, 16, true, kLimbBatch>), grid, block, p.lds, stream, tiles,
                               x, op, m, l.n, l.k, l.kx, l.gp, l.nb);
        else
            hipLaunchKernelGGL((decode_limb_rows_kernel<8, 2, 16, true, kLimbBatch>), grid, block, p.lds, stream, tiles,
                               x, op, m, l.n, l.k, l.kx, l.gp, l.nb);
    } else if (mt == 4) {
        if (!p.c.strided)
            Q4_LR(4, 2, 16, false);
        else if (p.c.waves == 16)
            Q4_LR(4, 1, 16, true);
        else
            Q4_LR(4, 2, 8, true);
    } else {
        if (!p.c.strided)
            Q4_LR(8, 2, 16, false);
        else if (p.c.waves == 16)
            Q4_LR(8, 2, 16, true);
        else
            Q4_LR(8, 2, 8, true);
    }
#undef Q4_LR
    return hipGetLastError();
}

hipError_t launch_decode_limbs(const uint4* tiles, const uint16_t* x, const OutParams& op, const Layout& l,
                               hipStream_t stream) {
    const size_t lds = limb_lds_bytes(l);
    if (lds > (size_t)160 * 1024) return hipErrorInvalidValue;
    const LimbConfig c = limb_config(l);
    const dim3 grid(limb_grid(l, c)), block(64 * c.waves);
    if (c.waves == 16)
        hipLaunchKernelGGL((decode_limb_kernel<3, 16, false>), grid, block, lds, stream, tiles, x, op, l.n, l.k, l.kx,
                           l.gp, l.nb);
    else if (!c.strided)
        hipLaunchKernelGGL((decode_limb_kernel<2, 8, false>), grid, block, lds, stream, tiles, x, op, l.n, l.k, l.kx,
                           l.gp, l.nb);
    else
        hipLaunchKernelGGL((decode_limb_kernel<1, 8, true>), grid, block, lds, stream, tiles, x, op, l.n, l.k, l.kx,
                           l.gp, l.nb);
    return hipGetLastError();
}

}  // namespace q4
