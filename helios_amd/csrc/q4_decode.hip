// Decode-shape affine-Q4 matmul on gfx950: y[M,N] = x[M,K] . W^T for M < 32 (and
// beyond, for weights small enough that slabs beat the GEMM's fixed costs), in
// 16-row slabs (one launch; slab = blockIdx.y).
//
// Bandwidth-bound: every weight byte is read once from HBM with 16-byte coalesced
// loads (one 1 KiB tile per wave-load, its scale/bias words right after it in the
// same record), scales/biases once per group, nibbles are
// expanded in registers (two VALU ops per bf16 pair) and the products run on the
// matrix cores: per group, two v_mfma_f32_16x16x32_bf16 give -X_g (x times a
// constant -1 operand, already in the accumulator layout) and two more give
// sum(x*(1+q/16)) - X_g seeded from it; the group's scale and bias are then applied
// to the fp32 accumulators (q4_common.h).  M is padded to 16 inside the MFMA, which
// costs nothing here: the matrix cores are far from busy at this arithmetic
// intensity, and the VALU work per weight stays at ~1.2 ops.
//
// Three kernels, chosen per shape in launch_mt: decode_kernel (one workgroup per
// 16-row block, its waves split the group pairs of K and meet in LDS for a split-K
// sum: no atomics, no second pass), decode_stream_kernel (the same split, persistent
// workgroups walking row blocks) and decode_rows_kernel (M = 1: one wave per row
// block).
#include <atomic>

#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

// Lane l of a 16x16 accumulator holds rows 4*(l/16)+r (r < 4) of column l%16, and
// row i of an MFMA result depends only on row i of its A operand, so A rows >= M
// may hold anything: they only feed accumulator rows that are never stored.
//
// XLDS = true (x[M,K] up to 64 KiB): the workgroup copies x into LDS, so the x
// operands cost LDS reads instead of a chain of L2 round trips.  XLDS = false (M up
// to 16): each wave reads its x operands from global memory, one group pair ahead.
//
// GPW: group pairs a wave handles per pass.  All of a pass's weight tiles and
// scales are requested before any arithmetic (GPW KiB in flight per wave, one HBM
// round trip).  Loads are bounded buffer loads, so pairs past the wave's range read
// as zero without branches; zero tiles with zero scale/bias add nothing.
template <int MT, int GPW, bool XLDS>
__global__ __launch_bounds__(1024) void decode_kernel(
    const uint4* __restrict__ tiles, const uint2* __restrict__ sb, const uint16_t* __restrict__ x_in,
    OutParams op_in, int m_total, int n_rows, int k, int kx, int gpairs, int waves) {
    constexpr int R = MT < 4 ? MT : 4;
    extern __shared__ uint4 xs_lds[];  // XLDS: x[M][K] as bf16, 16 B per entry
    // this workgroup's 16-row slab (blockIdx.y) of the launch's m_total rows
    const int slab = (int)blockIdx.y;
    const int m_rows = m_total - 16 * slab < 16 ? m_total - 16 * slab : 16;
    const uint16_t* __restrict__ x = x_in + (size_t)slab * 16 * kx;
    const OutParams op = slab_params(op_in, slab, n_rows);
    const int rb = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int gp0 = (wave * gpairs) / waves;
    const int cnt = ((wave + 1) * gpairs) / waves - gp0;
    const uint32_t xbytes = (uint32_t)m_rows * (uint32_t)k * 2u;  // of x' (rows of k)
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)kx * 2u);
    const int arow = col < m_rows ? col : m_rows - 1;  // any valid row for A rows >= M
    const uint32_t lane_x = (uint32_t)(arow * kx + 8 * kq) * 2u;  // XLDS = false: this lane's x bytes

    // a pass's tiles and scales as bounded buffers: pairs i >= left read as zero
    uint4 wv[GPW];
    uint2 sv[GPW];
    auto issue = [&](int base) {
        const int left = cnt - base;
        const long first = (long)rb * gpairs + gp0 + base;
        const __amdgpu_buffer_rsrc_t trs = make_rsrc(tiles + first * kRecU4, (uint32_t)left * kRecBytes);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb + first * kRecU2, sb_span(left));
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            wv[i] = buffer_load16<kNonTemporal>(trs, (uint32_t)(lane * 16 + i * kRecBytes));
            sv[i] = buffer_load8<kNonTemporal>(srs, (uint32_t)(col * 8 + i * kRecBytes));
        }
    };
    // XLDS = false: the first pass's weights are requested before anything else
    // (q_proj 4096x3840 at M = 16: 8.2 -> 6.8 us, the full-attention o 3840x8192 at
    // M = 4 and 8: 8.9 -> 7.8, 9.8 -> 8.6).  XLDS = true keeps them after the copy of
    // x: issued before it, each wave's x loads complete behind its weight loads and
    // the barrier after the copy waits for every wave's weights (q_proj at M = 1-8
    // 3-11% slower, qkv 13-19%).
    // (Not at M = 1 with 8-pair passes: held across the pass loop, those loads take it
    // past the 128 VGPRs of a 1024-thread workgroup, into scratch.)
    constexpr bool kIssueFirst = !XLDS && !(MT == 1 && GPW == 8);
    if (kIssueFirst && cnt > 0) issue(0);

    if constexpr (XLDS) {
        // cooperative copy x -> LDS
        const int chunks = (int)(xbytes >> 4);
        const int nthr = waves * 64;
        // eight units per thread in flight (x of 8 rows x 3840 on 512 threads is 7.5),
        // so the copy is one round trip
        constexpr int kCopy = 8;
        uint4 tmp[kCopy];
        for (int c0 = 0; c0 < chunks; c0 += kCopy * nthr) {
#pragma unroll
            for (int u = 0; u < kCopy; ++u) {
                const int c = c0 + u * nthr + (int)threadIdx.x;
                tmp[u] = buffer_load16(xrs, c < chunks ? xprime_offset(c, k, kx) : kOutOfRange);
            }
#pragma unroll
            for (int u = 0; u < kCopy; ++u) {
                const int c = c0 + u * nthr + (int)threadIdx.x;
                if (c < chunks) xs_lds[c] = tmp[u];
            }
        }
    }

    const uint4 neg1_bits = make_uint4(0xBF80BF80u, 0xBF80BF80u, 0xBF80BF80u, 0xBF80BF80u);
    const bf16x8 neg1 = __builtin_bit_cast(bf16x8, neg1_bits);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc = zero;
    bool synced = !XLDS;

    for (int base = 0; base < cnt; base += GPW) {
        const int gpb = gp0 + base;
        const int left = cnt - base;
        // element offset of this lane's x operand at pair i, group 0, half 0 (x in LDS)
        const int xel = arow * k + 8 * kq + gpb * 128;
        const int kleft = k - gpb * 128;

        if (!kIssueFirst || base > 0) issue(base);
        if (!synced) {
            __syncthreads();  // x is in LDS
            synced = true;
        }

        // x operands for one group pair: [group][half]; columns past the row (padding
        // or beyond this pass's pairs) read as zero.  kAhead pairs are in flight: from
        // L2 (XLDS = false) each is a round trip, and 8-pair passes chain eight
        constexpr int kAhead = !XLDS && GPW == 8 ? 2 : 1;
        uint4 a[kAhead + 1][4];
        auto load_x = [&](uint4* dst, int i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int kb = i * 128 + (q >> 1) * 64 + (q & 1) * 32;
                const bool ok = kb < kleft && i < left;
                if constexpr (XLDS) {
                    dst[q] = ok ? xs_lds[(xel + kb) >> 3] : make_uint4(0, 0, 0, 0);
                } else {
                    // a per-lane offset plus the operand's wave-uniform column (in the
                    // scalar offset): column cu of x' is column cu mod kx of x
                    const int cu = gpb * 128 + kb;
                    const int cm = cu >= kx ? cu - kx : cu;
                    dst[q] = buffer_load16s(xrs, ok ? lane_x : kOutOfRange, (uint32_t)cm * 2u);
                }
            }
        };
#pragma unroll
        for (int i = 0; i < kAhead; ++i) load_x(a[i], i);

#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            if (i + kAhead < GPW) load_x(a[(i + kAhead) % (kAhead + 1)], i + kAhead);
            const uint4* ax = a[i % (kAhead + 1)];
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                const bf16x8 x0 = __builtin_bit_cast(bf16x8, ax[2 * gi]);
                const bf16x8 x1 = __builtin_bit_cast(bf16x8, ax[2 * gi + 1]);
                f32x4 xn = mfma16x16x32(x0, neg1, zero);
                xn = mfma16x16x32(x1, neg1, xn);  // -X_g for rows 4*kq + r
                const bf16x8 b0 = expand_word(gi ? wv[i].z : wv[i].x);
                const bf16x8 b1 = expand_word(gi ? wv[i].w : wv[i].y);
                f32x4 p = mfma16x16x32(x0, b0, xn);
                p = mfma16x16x32(x1, b1, p);  // sum(x*q)/16
                const uint32_t sbv = gi ? sv[i].y : sv[i].x;
                const float s16 = bf16_lo(sbv) * 16.0f;
                const float bi = bf16_hi(sbv);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    acc[r] = __builtin_fmaf(s16, p[r], acc[r]);
                    acc[r] = __builtin_fmaf(-bi, xn[r], acc[r]);
                }
            }
        }
    }
    if (!synced) __syncthreads();  // (cnt == 0) keep barriers uniform

    __shared__ float red[16][R * 64];
#pragma unroll
    for (int r = 0; r < R; ++r) red[wave][r * 64 + lane] = acc[r];
    __syncthreads();
    for (int t = threadIdx.x; t < R * 64; t += waves * 64) {
        float v = 0.f;
        for (int w = 0; w < waves; ++w) v += red[w][t];
        const int r = t >> 6;
        const int l = t & 63;
        store_out(op, 4 * (l >> 4) + r, m_rows, rb, l & 15, n_rows, v);
    }
}

// A chunk's scale/bias words (4 pairs x 16 columns x 8 bytes, contiguous) arrive with
// one 8-byte load per lane: lane (col, kq) holds pair kq of column col.  Pair i of a
// lane's own column is fetched from lane 16 i + col through the LDS crossbar.  (Four
// loads of 8 bytes, each address shared by 4 lanes, cost the memory pipeline about
// 13% of the lm_head's time; permutes do not touch it.)
__device__ __forceinline__ uint32_t scale_word(uint2 sv, int pair, int gi, int col) {
    const int src = (16 * pair + col) * 4;
    return (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(gi ? sv.y : sv.x));
}

// Persistent streaming variant (x staged in LDS, up to 16 rows per slab).  Each
// workgroup walks row blocks blockIdx.x, blockIdx.x + gridDim.x, ...; its waves split K and stream
// their weight tiles in chunks of GPW group pairs, NBUF chunks in flight (two, or
// four for long walks at one workgroup per CU), so the loads for the next chunks
// (possibly of the next row blocks) are in flight while the current one is
// multiplied.  Per workgroup, once:
//   * x[M][K] is copied to LDS, each row zero-padded by GPW pairs so that operand
//     reads need no bounds tests (zero tiles past a wave's range meet finite x), and
//     one 16-byte unit more so that rows sit an odd number of units apart (the 16
//     rows of an operand read then fall in different banks);
//   * -X_g (the group sums of x, negated) is summed while x is copied and kept in
//     LDS in accumulator layout, so each row block needs only the two products of
//     the group, seeded from that table.  Table rows >= M are never written: they
//     only reach accumulator rows that are never stored.
// Per row block the waves meet once in LDS (ping-pong buffers, one barrier).
template <int MT, int GPW, int NBUF>
__global__ __launch_bounds__(512) void decode_stream_kernel(
    const uint4* __restrict__ tiles, const uint2* __restrict__ sb, const uint16_t* __restrict__ x_in,
    OutParams op_in, int m_total, int n_rows, int k, int kx, int gpairs, int nblocks, int waves) {
    constexpr int R = MT < 4 ? MT : 4;
    constexpr int kPad = GPW * 128;  // zero columns after each x row
    extern __shared__ uint4 lds[];
    // this workgroup's 16-row slab (blockIdx.y) of the launch's m_total rows
    const int slab = (int)blockIdx.y;
    const int m_rows = m_total - 16 * slab < 16 ? m_total - 16 * slab : 16;
    const uint16_t* __restrict__ x = x_in + (size_t)slab * 16 * kx;
    const OutParams op = slab_params(op_in, slab, n_rows);
    // layout: x rows [m_rows][k + kPad + 8] bf16, then -X table [2*(gpairs+GPW)][16] fp32
    __shared__ float red[2][8][R * 64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int gp0 = (wave * gpairs) / waves;
    const int cnt = ((wave + 1) * gpairs) / waves - gp0;  // >= 1 (host: waves <= gpairs)
    const int passes = (cnt + GPW - 1) / GPW;
    const int my_blocks = (nblocks - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int chunks = my_blocks * passes;
    const int arow = col < m_rows ? col : m_rows - 1;  // any valid row for A rows >= M
    // x row stride in 16-byte units: odd (one unit past the padding), so the 16 rows
    // one operand read touches fall in different LDS banks
    const int row16 = ((k + kPad) >> 3) + 1;
    const int groups = k >> 6;
    float* negx = reinterpret_cast<float*>(lds + m_rows * row16);  // [2 * (gpairs + GPW)][16]

    static_assert(GPW == 4, "one 8-byte load per lane covers a chunk's scale words");
    uint4 w[NBUF][GPW];
    uint2 sv[NBUF];  // scale words of a chunk: lane (col, kq) holds pair kq, column col
    // Chunks past the workgroup's last are issued too, against an empty range (zeros,
    // no memory traffic): every loop iteration then issues the same loads, which keeps
    // the compiler's wait counts exact (a conditional issue makes it wait for both
    // buffers before using either, draining the prefetch).
    auto issue = [&](uint4* wv, uint2& sv, int c) {
        const bool live = c < chunks;
        const int rb = live ? (int)blockIdx.x + (c / passes) * (int)gridDim.x : 0;
        const int pass = c % passes;
        const int gpb = gp0 + pass * GPW;
        const int left = cnt - pass * GPW;
        const int n_in = !live ? 0 : left < GPW ? left : GPW;
        const long first = (long)rb * gpairs + gpb;
        const __amdgpu_buffer_rsrc_t trs = make_rsrc(tiles + first * kRecU4, (uint32_t)n_in * kRecBytes);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb + first * kRecU2, sb_span(n_in));
#pragma unroll
        for (int i = 0; i < GPW; ++i) wv[i] = buffer_load16<kNonTemporal>(trs, (uint32_t)(lane * 16 + i * kRecBytes));
        // lane (col, kq): pair kq's word for row col
        sv = buffer_load8<kNonTemporal>(srs, (uint32_t)((lane >> 4) * kRecBytes + (lane & 15) * 8));
    };

    // x -> LDS (loads issued before any weight load), zero padding after each row,
    // and -X_g for every (group, row) into the table: each thread sums its eight
    // values, eight consecutive lanes hold one group (K/8 is a multiple of 8)
    {
        const int xchunks = (m_rows * k) >> 3;
        const int rowc = k >> 3;
        const int nthr = waves * 64;
        const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)kx * 2u);
        // up to kXB batches of four x units per thread are requested before the weights
        // (loads complete in order: x requested after them waits for every weight load
        // in flight); 16 rows of K = 3840 take 15 units per thread of 512
        constexpr int kXB = 4;
        uint4 tmp[kXB][4];
        auto load_x = [&](uint4* t, int c0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * nthr + (int)threadIdx.x;
                t[u] = buffer_load16(xrs, c < xchunks ? xprime_offset(c, k, kx) : kOutOfRange);
            }
        };
        auto store_x = [&](const uint4* t, int c0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * nthr + (int)threadIdx.x;
                const int row = c / rowc;
                const int cr = c - row * rowc;
                if (c < xchunks) lds[row * row16 + cr] = t[u];
                const uint32_t w4[4] = {t[u].x, t[u].y, t[u].z, t[u].w};
                float sum = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j) sum += bf16_lo(w4[j]) + bf16_hi(w4[j]);
                sum = octet_sum(sum);
                if (c < xchunks && (lane & 7) == 0) negx[(cr >> 3) * 16 + row] = -sum;
            }
        };
        // the first batches of x, then every weight buffer, then the batches are stored:
        // in straight-line code, so waiting for x leaves the weight loads in flight
        const int xb = (xchunks + 4 * nthr - 1) / (4 * nthr) < kXB ? (xchunks + 4 * nthr - 1) / (4 * nthr) : kXB;
#pragma unroll
        for (int b = 0; b < kXB; ++b)
            if (b == 0 || b < xb) load_x(tmp[b], b * 4 * nthr);
#pragma unroll
        for (int b = 0; b < NBUF; ++b) issue(w[b], sv[b], b);
#pragma unroll
        for (int b = 0; b < kXB; ++b)
            if (b == 0 || b < xb) store_x(tmp[b], b * 4 * nthr);
        for (int c0 = kXB * 4 * nthr; c0 < xchunks; c0 += 4 * nthr) {  // rows past 8192 elements per thread
            load_x(tmp[0], c0);
            store_x(tmp[0], c0);
        }
        for (int c = threadIdx.x; c < m_rows * (kPad >> 3); c += nthr)
            lds[(c / (kPad >> 3)) * row16 + rowc + (c % (kPad >> 3))] = make_uint4(0, 0, 0, 0);
        // table entries of groups past K (padding, and pairs past a wave's range) are
        // read by zero weight slots: they must be finite, so zero them
        for (int t = groups * 16 + (int)threadIdx.x; t < 2 * (gpairs + GPW) * 16; t += nthr) negx[t] = 0.f;
    }
    __syncthreads();

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc = zero;
    int parity = 0;
    auto compute = [&](const uint4* wv, const uint2 sv, int c) {
        const int pass = c % passes;
        const int gpb = gp0 + pass * GPW;
        const uint4* xp = lds + arow * row16 + kq + gpb * 16;  // x operand, pair 0
        const float* np = negx + gpb * 32 + 4 * kq;              // -X table, pair 0
        // operands are read per product (not gathered for the whole chunk first): this
        // keeps the kernel within 128 VGPRs, so two 8-wave workgroups fit on a CU
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                const bf16x8 xo0 = __builtin_bit_cast(bf16x8, xp[i * 16 + gi * 8]);
                const bf16x8 xo1 = __builtin_bit_cast(bf16x8, xp[i * 16 + gi * 8 + 4]);
                f32x4 xn;
                if constexpr (R == 1) {
                    xn = zero;
                    xn[0] = np[i * 32 + gi * 16];
                } else {
                    xn = *reinterpret_cast<const f32x4*>(np + i * 32 + gi * 16);
                }
                const uint32_t sbw = scale_word(sv, i, gi, col);
                const bf16x8 b0 = expand_word(gi ? wv[i].z : wv[i].x);
                const bf16x8 b1 = expand_word(gi ? wv[i].w : wv[i].y);
                f32x4 p = mfma16x16x32(xo0, b0, xn);
                p = mfma16x16x32(xo1, b1, p);  // sum(x*q)/16
                const float s16 = bf16_lo(sbw) * 16.0f;
                const float bi = bf16_hi(sbw);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    acc[r] = __builtin_fmaf(s16, p[r], acc[r]);
                    acc[r] = __builtin_fmaf(-bi, xn[r], acc[r]);
                }
            }
        }
        if (pass == passes - 1) {  // row block done: split-K sum across the waves
            const int rb = (int)blockIdx.x + (c / passes) * (int)gridDim.x;
#pragma unroll
            for (int r = 0; r < R; ++r) red[parity][wave][r * 64 + lane] = acc[r];
            __syncthreads();
            for (int t = threadIdx.x; t < R * 64; t += waves * 64) {
                float v = 0.f;
                for (int w = 0; w < waves; ++w) v += red[parity][w][t];
                const int r = t >> 6;
                const int l = t & 63;
                store_out(op, 4 * (l >> 4) + r, m_rows, rb, l & 15, n_rows, v);
            }
            acc = zero;
            parity ^= 1;
        }
    };

    // NBUF chunks in flight: compute one buffer, then refill it NBUF chunks ahead
    int c = 0;
    for (; c + NBUF <= chunks; c += NBUF) {
#pragma unroll
        for (int b = 0; b < NBUF; ++b) {
            compute(w[b], sv[b], c + b);
            issue(w[b], sv[b], c + b + NBUF);
        }
    }
#pragma unroll
    for (int b = 0; b + 1 < NBUF; ++b)  // fewer than NBUF chunks remain
        if (c + b < chunks) compute(w[b], sv[b], c + b);
}

// Row-block-per-wave variant, launched for M = 1 when N has many row blocks (gate
// and the gate|up pair).  Every wave owns whole 16-row blocks (wave w of the grid takes blocks w,
// w + total waves, ...), so there is no cross-wave reduction and no barrier after x
// is staged, and each wave keeps NBUF chunks of GPW tiles in flight across block
// boundaries.  x is staged in LDS once per workgroup, with the table of -X_g per
// (group, row) that seeds the MFMAs as in decode_stream_kernel.  (At M = 1 a VALU
// path with v_dot2_f32_bf16 was measured too: it issues as many cycles per chunk as
// the 16x16x32 MFMAs it replaces and was slower on the lm_head, so the matrix cores
// stay.)
template <int MT, int GPW, int NBUF>
__global__ __launch_bounds__(256) void decode_rows_kernel(
    const uint4* __restrict__ tiles, const uint2* __restrict__ sb, const uint16_t* __restrict__ x,
    OutParams op, int m_rows, int n_rows, int k, int kx, int gpairs, int nblocks) {
    static_assert(GPW == 4, "one 8-byte load per lane covers a chunk's scale words");
    constexpr int R = MT < 4 ? MT : 4;
    constexpr int kPad = GPW * 128;  // zero columns after each x row
    extern __shared__ uint4 lds[];
    const int waves = (int)(blockDim.x >> 6);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int gwave = (int)blockIdx.x * waves + wave;
    const int nwaves = (int)gridDim.x * waves;
    const int passes = (gpairs + GPW - 1) / GPW;
    const int my_blocks = gwave < nblocks ? (nblocks - gwave + nwaves - 1) / nwaves : 0;
    const int chunks = my_blocks * passes;
    const int arow = col < m_rows ? col : m_rows - 1;  // any valid row for A rows >= M
    const int row16 = (k + kPad) >> 3;                 // x row stride in 16-byte units
    const int groups = k >> 6;
    // -X_g table [2 * (gpairs + GPW)][16]
    float* xtab = reinterpret_cast<float*>(lds + m_rows * row16);

    uint4 w[NBUF][GPW];
    uint2 sv[NBUF];  // scale words of a chunk: lane (col, kq) holds pair kq, column col
    // chunk c: block (c / passes), pairs [GPW * (c % passes), ...).  Chunks past the
    // wave's last read an empty range (zeros, no traffic): every loop iteration issues
    // the same loads, which keeps the compiler's wait counts exact.
    auto issue = [&](int b, int c) {
        const bool live = c < chunks;
        const int rb = live ? gwave + (c / passes) * nwaves : 0;
        const int gpb = (c % passes) * GPW;
        const int left = gpairs - gpb;
        const int n_in = !live ? 0 : left < GPW ? left : GPW;
        const long first = (long)rb * gpairs + gpb;
        const __amdgpu_buffer_rsrc_t trs = make_rsrc(tiles + first * kRecU4, (uint32_t)n_in * kRecBytes);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb + first * kRecU2, sb_span(n_in));
#pragma unroll
        for (int i = 0; i < GPW; ++i) w[b][i] = buffer_load16<kNonTemporal>(trs, (uint32_t)(lane * 16 + i * kRecBytes));
        // lane (col, kq): pair kq's word for row col
        sv[b] = buffer_load8<kNonTemporal>(srs, (uint32_t)((lane >> 4) * kRecBytes + (lane & 15) * 8));
    };

    // x -> LDS with zero padding after each row, and -X_g into the table; the first
    // batch of x is requested before the weights
    {
        const int xchunks = (m_rows * k) >> 3;
        const int rowc = k >> 3;
        const int nthr = waves * 64;
        const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)kx * 2u);
        uint4 tmp[4];
        auto load_x = [&](int c0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * nthr + (int)threadIdx.x;
                tmp[u] = buffer_load16(xrs, c < xchunks ? xprime_offset(c, k, kx) : kOutOfRange);
            }
        };
        // each thread sums its eight values; eight consecutive lanes hold one group
        // (K/8 is a multiple of 8)
        auto store_x = [&](int c0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * nthr + (int)threadIdx.x;
                const int row = c / rowc;
                const int cr = c - row * rowc;
                if (c < xchunks) lds[row * row16 + cr] = tmp[u];
                const uint32_t w4[4] = {tmp[u].x, tmp[u].y, tmp[u].z, tmp[u].w};
                float sum = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j) sum += bf16_lo(w4[j]) + bf16_hi(w4[j]);
                sum = octet_sum(sum);
                if (c < xchunks && (lane & 7) == 0) xtab[(cr >> 3) * 16 + row] = -sum;
            }
        };
        load_x(0);
#pragma unroll
        for (int b = 0; b < NBUF; ++b) issue(b, b);
        store_x(0);
        for (int c0 = 4 * nthr; c0 < xchunks; c0 += 4 * nthr) {
            load_x(c0);
            store_x(c0);
        }
        for (int c = threadIdx.x; c < m_rows * (kPad >> 3); c += nthr)
            lds[(c / (kPad >> 3)) * row16 + rowc + (c % (kPad >> 3))] = make_uint4(0, 0, 0, 0);
        // table entries of groups past K are read with zero weight slots: keep them finite
        const int tab_used = groups * 16, tab_all = 2 * (gpairs + GPW) * 16;
        for (int t = tab_used + (int)threadIdx.x; t < tab_all; t += nthr) xtab[t] = 0.f;
    }
    __syncthreads();

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc = zero;
    auto compute = [&](int b, int c) {
        const int pass = c % passes;
        const int gpb = pass * GPW;
        const uint4* xp = lds + arow * row16 + kq + gpb * 16;  // x operand, pair 0
        // every LDS operand of the chunk first (x, table, scale words), so their latency
        // is paid once per chunk rather than before each product
        bf16x8 xo[GPW][2][2];
        f32x4 xn[GPW][2];
        uint32_t sbw[GPW][2];
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                xo[i][gi][0] = __builtin_bit_cast(bf16x8, xp[i * 16 + gi * 8]);
                xo[i][gi][1] = __builtin_bit_cast(bf16x8, xp[i * 16 + gi * 8 + 4]);
                // whole 16-byte table entries even at M = 1: rows >= M of the table are
                // never written, but they only seed accumulator rows that are never
                // stored, and a full read saves the three moves that zero them
                xn[i][gi] = *reinterpret_cast<const f32x4*>(xtab + (gpb + i) * 32 + gi * 16 + 4 * kq);
                sbw[i][gi] = scale_word(sv[b], i, gi, col);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the gather ahead of the math
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                const bf16x8 b0 = expand_word(gi ? w[b][i].z : w[b][i].x);
                const bf16x8 b1 = expand_word(gi ? w[b][i].w : w[b][i].y);
                const float s16 = bf16_lo(sbw[i][gi]) * 16.0f;
                const float bi = bf16_hi(sbw[i][gi]);
                f32x4 p = mfma16x16x32(xo[i][gi][0], b0, xn[i][gi]);
                p = mfma16x16x32(xo[i][gi][1], b1, p);  // sum(x*q)/16
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    acc[r] = __builtin_fmaf(s16, p[r], acc[r]);
                    acc[r] = __builtin_fmaf(-bi, xn[i][gi][r], acc[r]);
                }
            }
        }
        if (pass == passes - 1) {  // block done
            const int rb = gwave + (c / passes) * nwaves;
            // lane holds rows 4*kq + r of column col
#pragma unroll
            for (int r = 0; r < R; ++r) store_out<false>(op, 4 * kq + r, m_rows, rb, col, n_rows, acc[r]);
            acc = zero;
        }
    };

    int c = 0;
    for (; c + NBUF <= chunks; c += NBUF) {
#pragma unroll
        for (int b = 0; b < NBUF; ++b) {
            compute(b, c + b);
            issue(b, c + b + NBUF);
        }
    }
#pragma unroll
    for (int b = 0; b < NBUF; ++b)
        if (c + b < chunks) compute(b, c + b);
}

// Split of K's group pairs over the waves of a workgroup: an exact GPW x waves
// factorisation when one exists (no zero passes), else 4 pairs per pass.  GPW = 6
// only fits the 128-VGPR budget (16 waves per workgroup) for M <= 2.
struct Split {
    int gpw;
    int waves;
};

inline Split choose_split(int gpairs, int mt) {
    if (mt <= 2 && gpairs % 6 == 0 && gpairs / 6 <= 16) return {6, gpairs / 6};
    if (gpairs % 4 == 0 && gpairs / 4 <= 16) return {4, gpairs / 4};
    // one pass of 8 pairs per wave (down_proj's 120 pairs: 15 waves) beats two passes
    // of 4 by 0.4-1.2 us at M = 5-16
    if (gpairs % 8 == 0 && gpairs / 8 <= 16) return {8, gpairs / 8};
    const int waves = (gpairs + 3) / 4 < 16 ? (gpairs + 3) / 4 : 16;
    return {4, waves};
}

constexpr size_t kLdsPerCu = 160 * 1024;  // gfx950 LDS per CU (and per workgroup)
// row-block-per-wave kernel: M = 1 and 2 with this many 16-row blocks, 4 waves per
// workgroup, at most this many workgroups per CU.  Measured against the other
// kernels: at M = 1 ~0.4 us ahead for gate (960 blocks) and gate|up (1920), 1.8% for
// the lm_head's 16384 (91.6 vs 93.3 us); at M = 2 gate 10.6 vs 11.35 us, gate|up
// 15.5 vs 17.4, the lm_head 92.1 vs 94.6; behind for the qkv-sized 512 blocks (9.2 vs
// 6.4 us at M = 1) and from M = 3 on (gate 12.9 vs 11.9 at M = 3, 13.7 vs 12.0 at 4).
constexpr int kRowsMinBlocks = 768;
constexpr int kRowsMaxBlocks = 16384;
// at M = 2 only up to this many group pairs of K (the measured gains above are at 30
// pairs); with 60 pairs (8-bit gate and gate|up pair) the row kernel and streaming
// were within the spread between machines (6-7% behind on one, 3-7% ahead on
// another), so those keep streaming
constexpr int kRowsM2MaxPairs = 32;
constexpr int kRowsWaves = 4;
constexpr int kRowsPerCu = 2;
// one workgroup per row block with x staged in LDS (decode_kernel<MT, 4, true>, 8
// waves of 4 pairs, one pass): for K of at most 32 pairs and up to this many row
// blocks (twice as many for M > 1) it is ahead of the streaming kernel (0.5-0.8 us at
// M = 1, 1-3 us at M = 8 for q/k/v/o and their fused qkv, 0.8 us for the qkv at
// M = 3-4); it is behind for the gate|up pair, the lm_head, down (K of 120 pairs) and
// gate at M = 1-2 (the row kernel's case).  For gate at M = 3-16 the two are within
// the spread between machines (streaming 6% ahead at M = 3-4 on one, 3% behind on
// another).
constexpr int kXLdsMaxPairs = 32;
constexpr int kXLdsMaxBlocks = 512;
constexpr size_t kXLdsMaxBytes = 64 * 1024;


// One launch over all m rows: slabs of 16 rows along the grid's y dimension (the
// workgroups of one row block in different slabs run close together, so the weights
// come from HBM about once).  MT = 16 whenever m > 16.
template <int MT>
hipError_t launch_mt(const uint4* tiles, const uint2* sb, const uint16_t* x, const OutParams& op, int m,
                     const Layout& l, hipStream_t stream) {
    constexpr int GPW = 4;
    constexpr int R = MT < 4 ? MT : 4;
    const int ms = m < 16 ? m : 16;  // rows per slab
    const unsigned slabs = (unsigned)((m + 15) / 16);
    const size_t static_lds = 2 * 8 * R * 64 * sizeof(float);
    const size_t lds_bytes = (size_t)ms * (l.k + GPW * 128) * 2 + (size_t)(l.gp + GPW) * 2 * 16 * 4;
    if constexpr (MT <= 2) {
        if (l.nb >= kRowsMinBlocks && l.nb <= kRowsMaxBlocks && lds_bytes <= kLdsPerCu && op.mode < kOutGreedyBf16 &&
            (MT == 1 || l.gp <= kRowsM2MaxPairs)) {
            // many row blocks: one wave per block, no cross-wave reduction
            int grid = (l.nb + kRowsWaves - 1) / kRowsWaves;
            const int cap = device_cus() * kRowsPerCu;
            if (grid > cap) grid = cap;
            hipLaunchKernelGGL((decode_rows_kernel<MT, GPW, 2>), dim3(grid), dim3(64 * kRowsWaves), lds_bytes, stream,
                               tiles, sb, x, op, m, l.n, l.k, l.kx, l.gp, l.nb);
            return hipGetLastError();
        }
    }
    const size_t x_bytes = (size_t)ms * l.k * 2;
    // K of at most 8 pairs (1024) from M = 5: two waves per row block, which cannot
    // cover staging x; the global-x kernel below is ahead (1024x1024 at M = 6 / 8 / 12 /
    // 16: 3.80 / 3.80 / 3.94 / 3.97 us against 4.05 / 4.11 / 4.40 / 4.70)
    const bool short_k = MT >= 8 && l.gp <= 8;
    if (!short_k && l.gp <= kXLdsMaxPairs && x_bytes <= kXLdsMaxBytes && l.nb <= kXLdsMaxBlocks * (MT > 1 ? 2 : 1)) {
        const int waves = (l.gp + GPW - 1) / GPW;  // <= 8, each wave one pass of <= 4 pairs
        hipLaunchKernelGGL((decode_kernel<MT, GPW, true>), dim3(l.nb, slabs), dim3(64 * waves), x_bytes, stream, tiles,
                           sb, x, op, m, l.n, l.k, l.kx, l.gp, waves);
        return hipGetLastError();
    }
    const size_t stream_lds = lds_bytes + (size_t)ms * 16;  // x rows one 16-byte unit longer
    // From M = 3, K too long for the per-row-block kernel but short enough for one pass
    // of at most 16 waves, the global-x variant below is ahead of streaming: K of a
    // multiple of 8 pairs beyond 64 (down_proj: 12.0 vs 12.6 us at M = 3, 12.5 vs 13.7
    // at 4; behind at M = 2), and K of 33-64 pairs in 4-pair waves when there are no
    // more row blocks than CUs (the full-attention o, 8192 x 240 blocks: 8.77 vs 9.08 at
    // M = 3, 8.92 vs 9.32 at 4; 8-bit q, 60 pairs x 256 blocks).  With more blocks
    // streaming stays ahead (8-bit gate, 960 blocks: 17.1 vs 28.1 us at M = 3; the
    // 8-bit gate|up pair and qkv likewise).
    const bool one_pass = MT >= 4 && ((l.gp % 8 == 0 && l.gp / 8 <= 16 && l.gp / 4 > 16) ||
                                      (l.gp > kXLdsMaxPairs && l.gp % 4 == 0 && l.gp / 4 <= 16 &&
                                       l.nb <= device_cus()));
    // persistent streaming kernel: 4 pairs per chunk, up to 8 waves per workgroup
    int waves = (l.gp + GPW - 1) / GPW;
    if (waves > 8) waves = 8;
    if (waves > l.gp) waves = l.gp;
    int per_cu = 20 / waves > 0 ? 20 / waves : 1;
    const int lds_fit = (int)(kLdsPerCu / (stream_lds + static_lds));
    if (per_cu > lds_fit) per_cu = lds_fit;
    const int capacity = device_cus() * (per_cu > 0 ? per_cu : 1);
    const int per_wg = (l.nb + capacity - 1) / capacity;
    // Slabs of 5-16 rows with one or two row blocks per workgroup: staging x (up to
    // 16 rows of K) costs each workgroup more than its weights, and the per-block
    // kernel below, reading x straight from L2, is ahead: q_proj 4096x3840 at M = 16
    // 7.7 vs 9.0 us, at M = 64 20.4 vs 31.6; k_proj 2048x3840 at M = 128 19.4 vs
    // 30.7; the fused qkv 8192x3840 (two blocks per workgroup) 20.9 vs 22.1 at M = 32,
    // and in one slab 9.8 vs 10.9 at M = 9-10, 11.3 vs 12.0 at 14, 12.0 vs 12.1 at 16
    // (but not its 8-bit twin, 60 pairs: streaming 13.9 / 15.3 vs 16.1 / 17.1 us at
    // M = 6 / 8).  gate 15360x3840 (four per workgroup) stays streaming: 15.4 vs 20.7
    // at M = 16.
    const bool few_blocks = MT == 16 && (per_wg == 1 || (per_wg == 2 && (slabs > 1 || l.gp <= kXLdsMaxPairs)));
    if (!one_pass && !few_blocks && !short_k && lds_fit > 0) {
        const int grid = (l.nb + per_wg - 1) / per_wg;
        // one workgroup per CU and a long walk (the lm_head at M = 8: 126 vs 135 us):
        // four chunks per wave in flight.  Not for short walks (down and the gate|up
        // pair at M = 2-16 were 5-15% slower: the deeper prefetch delays x staging).
        if (per_cu == 1 && per_wg >= 16)
            hipLaunchKernelGGL((decode_stream_kernel<MT, GPW, 4>), dim3(grid, slabs), dim3(64 * waves), stream_lds,
                               stream, tiles, sb, x, op, m, l.n, l.k, l.kx, l.gp, l.nb, waves);
        else
            hipLaunchKernelGGL((decode_stream_kernel<MT, GPW, 2>), dim3(grid, slabs), dim3(64 * waves), stream_lds,
                               stream, tiles, sb, x, op, m, l.n, l.k, l.kx, l.gp, l.nb, waves);
        return hipGetLastError();
    }
    const Split sp = choose_split(l.gp, MT);
    const dim3 grid(l.nb, slabs), block(64 * sp.waves);
    if (sp.gpw == 8)
        hipLaunchKernelGGL((decode_kernel<MT, 8, false>), grid, block, 0, stream, tiles, sb, x, op, m, l.n, l.k, l.kx, l.gp, sp.waves);
    else if (sp.gpw == 6)
        hipLaunchKernelGGL((decode_kernel<MT, 6, false>), grid, block, 0, stream, tiles, sb, x, op, m, l.n, l.k, l.kx, l.gp, sp.waves);
    else
        hipLaunchKernelGGL((decode_kernel<MT, 4, false>), grid, block, 0, stream, tiles, sb, x, op, m, l.n, l.k, l.kx, l.gp, sp.waves);
    return hipGetLastError();
}

}  // namespace

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev] = v;
    }
    return cus[dev];
}

namespace {
std::atomic<int> g_decode_variant{0};
}  // namespace

int set_decode_variant(int v) { return g_decode_variant.exchange(v); }
int decode_variant() { return g_decode_variant.load(std::memory_order_relaxed); }

hipError_t launch_decode(const uint4* tiles, const uint2* sb, const uint16_t* x, const OutParams& op, int m,
                         const Layout& l, hipStream_t stream) {
    const int variant = decode_variant();
    if (m == 1 && variant != 2 && limb_lds_bytes(l) <= kLdsPerCu) return launch_decode_limbs(tiles, x, op, l, stream);
    if (m >= 2 && m <= 8 && variant != 2 && (variant == 1 || limb_rows_preferred(l, m)) &&
        limb_rows_lds_bytes(l, m) <= kLdsPerCu)
        return launch_decode_limb_rows(tiles, x, op, m, l, stream);
    if (m == 1) return launch_mt<1>(tiles, sb, x, op, m, l, stream);
    if (m == 2) return launch_mt<2>(tiles, sb, x, op, m, l, stream);
    if (m <= 4) return launch_mt<4>(tiles, sb, x, op, m, l, stream);
    return launch_mt<16>(tiles, sb, x, op, m, l, stream);
}

// argmax over the blocks' best keys: one workgroup per row (deterministic: the max of
// keys does not depend on order)
__global__ __launch_bounds__(256) void greedy_reduce_kernel(const unsigned long long* __restrict__ part, int nb,
                                                            int32_t* __restrict__ token, float* __restrict__ value) {
    const int m = (int)blockIdx.x;
    unsigned long long best = 0;
    for (int i = (int)threadIdx.x; i < nb; i += (int)blockDim.x) {
        const unsigned long long k = part[(long)m * nb + i];
        best = k > best ? k : best;
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const unsigned long long o = __shfl_xor(best, d);
        best = o > best ? o : best;
    }
    __shared__ unsigned long long wbest[4];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) best = wbest[w] > best ? wbest[w] : best;
        token[m] = greedy_index(best);
        if (value != nullptr) value[m] = greedy_value(best);
    }
}

hipError_t launch_greedy_reduce(const unsigned long long* part, int nb, int m, int32_t* token, float* value,
                                hipStream_t stream) {
    hipLaunchKernelGGL(greedy_reduce_kernel, dim3(m), dim3(256), 0, stream, part, nb, token, value);
    return hipGetLastError();
}

}  // namespace q4
