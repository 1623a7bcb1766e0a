// Prefill-shape affine-Q4 matmul on gfx950: y[M,N] = x[M,K] . W^T for large M.
//
// Exact factored form on the matrix cores (q4_common.h):
//   y = sum_g 16*s_g * P_g + (b_g - 16*s_g) * X_g,   P_g = sum_{k in g} x*(1 + q/16)
// * P_g: two v_mfma_f32_16x16x32_bf16 per 16x16 tile per group, B operands expanded
//   from the tiled nibbles in registers (no dequantized weights anywhere), then
//   acc += 16*s * P_g on the fp32 accumulators (one VALU FMA per output per group);
// * the bias term: one extra MFMA per tile per 8 groups on an augmented K of 32,
//   A = [Xh, Xl, -16Xh, -16Xl] per group (X_g = Xh + Xl split into two bf16),
//   B = [b, b, s, s] taken straight from the scale/bias words.  In the 64- and
//   128-row tiles X_g comes from the x tile in LDS: two MFMAs of an all-ones A
//   against a row tile's x fragments (as B) sum the group's 64 values of its 16 rows,
//   each wave for its own row tiles.  The 256-row tile takes it from xaug_kernel, a
//   pre-pass: there every wave reads the 256 rows' fragments from LDS already (about
//   256 KiB per CU per group step), and reading them again cost more than the
//   pre-pass's launch (gate 15360x3840 at 2048 rows 228.5 -> 232.4 us).
// Every product is exact; rounding is fp32 accumulation only.
//
// The fp16 form (256-row tiles, when the handle's scales allow it): with
// s' = s 2^p and x scaled per row to x16 = fp16(x 2^k) by a pre-pass (xprep_kernel),
//   y 2^(k + p) = sum_k x16 * s'(q - 8) + sum_g X_g 2^p (b + 8 s),   X_g = sum of x16,
// where s'(q - 8) is exact in fp16 (q4_common.h) and every product is again exact:
// the matrix cores (v_mfma_f32_16x16x32_f16) accumulate straight into the outputs and
// the per-group scale FMAs go away (two per MFMA; with the expansion's four extra ops
// per word, 81 VALU ops per group step instead of ~240).  The bias term is the same
// MFMA with A = [Xh, Xl, 8Xh, 8Xl] (X_g 2^p).  x16 is exact for every x within 2^32 of
// its row's largest; smaller ones are rounded at 2^-39 of it.  The outputs are scaled
// back by 2^-(k + p) before any store.  Measured on gate 15360x3840 at 2048 rows
// (rocprof, steady clock): the GEMM kernel 210-215 us against 218-223 in the bf16
// form, but the pre-pass, which now writes x16 (15.7 MB), 12 us against 5; so the plan
// takes the form only where its cost model says the kernel's gain is larger (the
// widest outputs: the gate|up pair, gate and up from ~1024 rows).
//
// Tiling: a 512-thread workgroup computes a 256 (M) x 256 (N) tile as eight waves
// side by side along N, each all 256 rows x 32 columns (two waves per SIMD, so one's
// MFMA and LDS latencies are covered by the other's work); or 128 x 256, or 64 x 256
// (eight waves of 128 or 64 x 32).  A wave expands only its own two row blocks'
// nibbles and reads every x row of the tile from LDS: expansion is VALU work and was
// the wider cost (measured against 2 x 4 waves of BM/2 x 64, with bit-identical
// results: the 64-row tile 8-13% faster, the 128-row tile 3-9%, the 256-row tile
// 0-6%).  The kernel is written
// for tiles of BN = 128 too (four waves, 78 KiB of LDS: two workgroups per CU); a
// forced-plan sweep over the benchmark's shapes measured it within 6% of the two
// tiles above where it helped at all, so the plan does not use it.  Everything streams
// through LDS by direct-to-LDS buffer loads (no staging registers): per 64-wide group the x tile (rows swizzled so the MFMA
// operand reads are bank-conflict free), the group's weight words and scale words;
// the bias operands once per 8 groups.  The x ring has three slots, so each load has
// two steps of arithmetic to arrive in (two slots, one step, for the one-pass 8-bit
// form on 256-row tiles, whose weight slots hold both planes).
#include <type_traits>

#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

constexpr int kWN = 32;               // wave tile columns (the wave tile spans all BM rows)
constexpr int kNT = kWN / 16;         // 16x16 tiles per wave along N

typedef __attribute__((address_space(3))) void* lds_ptr_t;


// The bias MFMA's A operand for one 16-row tile and one octet, as 64 lanes of 16 B:
// lane (m = l%16, kq = l/16), element e -> group 8*octet + 2*kq + e/4, term e%4 in
// {Xh, Xl, c Xh, c Xl} (c = -16, or 8 in the fp16 form).  Lane (m, kq) packs it from X
// of row m for groups 2kq and 2kq + 1.
template <int C = -16>
__device__ __forceinline__ uint4 bias_a_operand(float x0, float x1) {
    uint32_t w[4];
    const float xs[2] = {x0, x1};
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const uint16_t xh = f32_to_bf16(xs[gi]);
        const uint16_t xl = f32_to_bf16(xs[gi] - __uint_as_float((uint32_t)xh << 16));
        const uint16_t nxh = f32_to_bf16((float)C * __uint_as_float((uint32_t)xh << 16));
        const uint16_t nxl = f32_to_bf16((float)C * __uint_as_float((uint32_t)xl << 16));
        w[2 * gi] = (uint32_t)xh | ((uint32_t)xl << 16);
        w[2 * gi + 1] = (uint32_t)nxh | ((uint32_t)nxl << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------
// X_g for the 256-row tile: bias A operands of every 16-row block and octet,
// xaug[m16][octet][lane] (16 B, as bias_a_operand).  One 512-thread workgroup per
// 1 KiB block (16 rows x one octet): eight lanes sum one (row, group) from its 128
// contiguous bytes, two rounds cover the 16 x 8 pairs, the sums meet in LDS and one
// wave packs the block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void xaug_kernel(const uint16_t* __restrict__ x, uint4* __restrict__ xaug,
                                                   int m_rows, int kx, int groups, int octets) {
    // x rows are kx long; group g >= kx / 64 (the low plane of a two-plane handle) is
    // group g - kx / 64 of x
    const int gx = kx >> 6;
    __shared__ float gsum[8][16];  // [group within the octet][row within the block]
    const int unit = (int)blockIdx.x;  // 16-row block * octets + octet
    const int o = unit % octets;
    const long mb = unit / octets;
    const int t = (int)threadIdx.x;
    const int c = t & 7;  // 16-byte chunk of the group
    uint4 v[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {  // both loads in flight before any sum
        const int p = (t >> 3) + 64 * r;
        const long m = mb * 16 + (p & 15);
        const int g = 8 * o + (p >> 4);
        v[r] = (m < m_rows && g < groups)
                   ? *reinterpret_cast<const uint4*>(x + m * kx + 64 * (g >= gx ? g - gx : g) + 8 * c)
                   : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int p = (t >> 3) + 64 * r;
        float sum = ((bf16_lo(v[r].x) + bf16_hi(v[r].x)) + (bf16_lo(v[r].y) + bf16_hi(v[r].y))) +
                    ((bf16_lo(v[r].z) + bf16_hi(v[r].z)) + (bf16_lo(v[r].w) + bf16_hi(v[r].w)));
        sum = octet_sum(sum);
        if (c == 0) gsum[p >> 4][p & 15] = sum;
    }
    __syncthreads();
    if (t >= 64) return;
    const int kq = t >> 4;
    xaug[(long)unit * 64 + t] = bias_a_operand(gsum[2 * kq][t & 15], gsum[2 * kq + 1][t & 15]);
}

// ---------------------------------------------------------------------------
// The fp16 form's pre-pass: one wave per row m of the tiles, four rows per workgroup
// (rows past M write zero bias operands only):
//  * k = 142 - e, e the largest biased exponent of the row's finite |x|, so that the
//    largest |x| 2^k lies in [2^15, 2^16), with 8 significant bits below 65504 (a row
//    whose finite values are all bf16 subnormals, e = 0: k = 142, and m 2^-133 2^142
//    = 512 m < 65504 is exact; k = 0 for a row of zeros; inf and NaN stay inf and NaN
//    and reach y so);
//  * x16[m] = fp16(x 2^k), exact for every x within 2^32 of the largest;
//  * X_g = the fp32 sum of the group's x16 values (in element order, then over the
//    group's eight 16-byte units in a fixed tree), and the 256-row tile's bias A
//    operands from X_g 2^p, in xaug_kernel's layout;
//  * rowexp[m] = k + p: the GEMM's sums of row m are y 2^(k + p).
// A lane keeps up to kPrepCache 16-byte units of its row between the two passes (rows
// of up to 4096 values are read once); longer rows are read again from L2.
// ---------------------------------------------------------------------------
constexpr int kPrepRows = 4;    // rows (waves) per workgroup
constexpr int kPrepCache = 8;

// largest bf16 magnitude bits of eight values, inf and NaN left out
__device__ __forceinline__ uint32_t finite_max_bits(uint4 v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t mb = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[j] & 0x7FFFu, hi = (w[j] >> 16) & 0x7FFFu;
        mb = (lo < 0x7F80u && lo > mb) ? lo : mb;
        mb = (hi < 0x7F80u && hi > mb) ? hi : mb;
    }
    return mb;
}

// C: the bias operand's factor (8 for the fp16 form; -64 for one-pass 8-bit, whose
// scale words hold 16 s: -64 * 16 s = -1024 s).
template <int C>
__global__ __launch_bounds__(64 * kPrepRows) void xprep_kernel(const uint16_t* __restrict__ x,
                                                               uint16_t* __restrict__ x16, uint4* __restrict__ xaug,
                                                               int* __restrict__ rowexp, int m_rows, int kx, int groups,
                                                               int octets, int p) {
    extern __shared__ float gsum_all[];  // [kPrepRows][kx / 64]
    const int wave = (int)(threadIdx.x >> 6);
    const int lane = (int)(threadIdx.x & 63);
    const int m = (int)blockIdx.x * kPrepRows + wave;
    const int gx = kx >> 6;     // groups of a row of x (a two-plane handle's group g >= gx is g - gx)
    const int units = kx >> 3;  // 16-byte units of the row (a multiple of 8)
    float* const gsum = gsum_all + wave * gx;
    if (m < m_rows) {
        const uint4* xr = reinterpret_cast<const uint4*>(x + (long)m * kx);
        uint4* yr = reinterpret_cast<uint4*>(x16 + (long)m * kx);
        const uint4 zero = make_uint4(0, 0, 0, 0);
        uint4 c[kPrepCache];
#pragma unroll
        for (int i = 0; i < kPrepCache; ++i) {
            const int u = lane + 64 * i;
            c[i] = u < units ? xr[u] : zero;
        }
        uint32_t mb = 0;
#pragma unroll
        for (int i = 0; i < kPrepCache; ++i) {
            const uint32_t v = finite_max_bits(c[i]);
            mb = v > mb ? v : mb;
        }
        for (int u = lane + 64 * kPrepCache; u < units; u += 64) {
            const uint32_t v = finite_max_bits(xr[u]);
            mb = v > mb ? v : mb;
        }
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_xor((int)mb, d);
            mb = o > mb ? o : mb;
        }
        const int e = (int)(mb >> 7);
        const int k = mb == 0 ? 0 : 142 - e;
        // x16 of one 16-byte unit and its group's sum (the eight units of a group are
        // eight consecutive lanes; every lane of the wave takes part in the shuffles)
        auto conv = [&](uint4 v, int u) {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t o[4];
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 lo = (_Float16)__builtin_amdgcn_ldexpf(bf16_lo(w[j]), k);
                const _Float16 hi = (_Float16)__builtin_amdgcn_ldexpf(bf16_hi(w[j]), k);
                sum += (float)lo;
                sum += (float)hi;
                o[j] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
            }
            sum = octet_sum(sum);
            if (u < units) {
                yr[u] = make_uint4(o[0], o[1], o[2], o[3]);
                if ((u & 7) == 0) gsum[u >> 3] = sum;
            }
        };
#pragma unroll
        for (int i = 0; i < kPrepCache; ++i)
            if (64 * i < units) conv(c[i], lane + 64 * i);
        for (int u0 = 64 * kPrepCache; u0 < units; u0 += 64) {
            const int u = u0 + lane;
            conv(u < units ? xr[u] : zero, u);
        }
        if (lane == 0) rowexp[m] = k + p;
    }
    __syncthreads();
    // entry (octet o, kq) of row m: groups 8o + 2kq and 8o + 2kq + 1
    const long m16 = m >> 4;
    const int r = m & 15;
    for (int i = lane; i < octets * 4; i += 64) {
        const int o = i >> 2, kq = i & 3;
        float xs[2];
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
            const int g = 8 * o + 2 * kq + gi;
            xs[gi] = (m < m_rows && g < groups) ? __builtin_amdgcn_ldexpf(gsum[g >= gx ? g - gx : g], p) : 0.0f;
        }
        xaug[(m16 * octets + o) * 64 + kq * 16 + r] = bias_a_operand<C>(xs[0], xs[1]);
    }
}

// Scale range of a handle: thread per (record, row), one atomic per wave.
__global__ void scale_range_kernel(const uint2* __restrict__ sb, long records, int* __restrict__ out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int emax = -1, emin = 255, bad = 0;  // (a subnormal scale counts as exponent 0)
    if (i < records * 16) {
        const uint2 w = sb[(i >> 4) * kRecU2 + (i & 15)];
        const uint32_t mags[2] = {w.x & 0x7FFFu, w.y & 0x7FFFu};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (mags[j] == 0) continue;
            const int e = (int)(mags[j] >> 7);
            if (e == 255) {
                ++bad;
            } else {
                emax = e > emax ? e : emax;
                emin = e < emin ? e : emin;
            }
        }
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int a = __shfl_xor(emax, d), b = __shfl_xor(emin, d), c = __shfl_xor(bad, d);
        emax = a > emax ? a : emax;
        emin = b < emin ? b : emin;
        bad += c;
    }
    if ((threadIdx.x & 63) == 0) {
        atomicMax(&out[0], emax);
        atomicMin(&out[1], emin);
        if (bad) atomicAdd(&out[2], bad);
    }
}

// B operand of the bias MFMA from one scale/bias word pair: [b0 b0 s0 s0 b1 b1 s1 s1]
__device__ __forceinline__ bf16x8 bias_operand(uint2 sbw) {
    uint4 d;
    d.x = __builtin_amdgcn_perm(sbw.x, sbw.x, 0x03020302u);  // b0 | b0 << 16
    d.y = __builtin_amdgcn_perm(sbw.x, sbw.x, 0x01000100u);  // s0 | s0 << 16
    d.z = __builtin_amdgcn_perm(sbw.y, sbw.y, 0x03020302u);
    d.w = __builtin_amdgcn_perm(sbw.y, sbw.y, 0x01000100u);
    return __builtin_bit_cast(bf16x8, d);
}

// Tile order: the hardware deals workgroup ids round-robin over the 8 XCDs; give
// each XCD a contiguous run of tiles, and walk tiles in bands of two M tiles
// (M fastest) so workgroups running together share x rows and weight tiles in L2.
__device__ __forceinline__ void tile_of(int id, int nwg, int mtiles, int ntiles, int& mt, int& nt) {
    constexpr int kXcds = 8;
    int tile = id;
    if (nwg % kXcds == 0) tile = (id % kXcds) * (nwg / kXcds) + id / kXcds;
    constexpr int kBand = 2;
    const int band = tile / (kBand * ntiles);
    const int r = tile - band * kBand * ntiles;
    const int bm = (mtiles - band * kBand) < kBand ? (mtiles - band * kBand) : kBand;
    mt = band * kBand + r % bm;
    nt = r / bm;
}

// t = x . A^T of a workgroup's BM rows into LDS (`ts`, [BM][rank] floats: the x ring's
// first slot, BM x 128 bytes, so rank <= 32), each entry summed over its slices in
// slice order; rows past the output read as zeros.  All of the workgroup's threads,
// one barrier after.
template <int BM>
__device__ __forceinline__ void lora_stage_t(const LoraEpilogue& lo, float* ts, int row0, int m_rows, int nthr) {
    const int q4s = lo.rank >> 2;  // float4s per row
    for (int t = (int)threadIdx.x; t < BM * q4s; t += nthr) {
        const int row = t / q4s, r = 4 * (t - row * q4s);
        const int m = row0 + row;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m < m_rows) {
            v = *reinterpret_cast<const float4*>(lo.part + (long)m * lo.rank + r);
            for (int sl = 1; sl < lo.slices; ++sl) {
                const float4 u = *reinterpret_cast<const float4*>(lo.part + ((long)sl * m_rows + m) * lo.rank + r);
                v.x = v.x + u.x;
                v.y = v.y + u.y;
                v.z = v.z + u.z;
                v.w = v.w + u.w;
            }
        }
        *reinterpret_cast<float4*>(ts + row * lo.rank + r) = v;
    }
    __syncthreads();
}

// Eight fp32 values as bf16 high parts and the bf16 roundings of what is left
// (v = hi + lo to about 2^-16 relative).
__device__ __forceinline__ void split_bf16x8(const float4 a, const float4 b, bf16x8& hi, bf16x8& lo) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const __bf16 h = (__bf16)v[e];
        hi[e] = h;
        lo[e] = (__bf16)(v[e] - (float)h);
    }
}

// The LoRA delta of a wave's output tiles and the combined store, in lora_up's
// rounding steps (q4_lora.hip): d[m, n] = sum_r t[m, r] B[n, r] on the bf16 matrix
// cores, t and B each split into bf16 high and low parts, d = th.bh + th.bl + tl.bh
// (three 16x16x32 MFMAs per tile cover every rank up to 32; the dropped tl.bl term and
// the parts' roundings leave d within about 2^-16 of the fp32 sum, far below the bf16
// rounding of the delta that follows); then y = bf16(bf16(acc) + bf16(d * bf16(scale)))
// in bf16, acc + d * scale in fp32.  Lane (row or column, kq) holds ranks 8kq..8kq+7;
// columns past the output and ranks past the adapter's read zeros.
template <bool F32, int kMT, int kNT>
__device__ __forceinline__ void lora_store(const f32x4 (&acc)[kMT][kNT], const LoraEpilogue& lo, const float* ts,
                                           void* y, int row0, int rb0, int m_rows, int n_rows, int lane) {
#pragma clang fp contract(off)
    const int col = lane & 15, kq = lane >> 4;
    const int r0 = 8 * kq;
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    bf16x8 bh[kNT], bl[kNT];
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
        const int n = (rb0 + j) * 16 + col;
        const bool ok = n < n_rows;
        const float* bp = lo.b + (long)(ok ? n : 0) * lo.rank + r0;
        const float4 b0 = ok && r0 < lo.rank ? *reinterpret_cast<const float4*>(bp) : zero4;
        const float4 b1 = ok && r0 + 4 < lo.rank ? *reinterpret_cast<const float4*>(bp + 4) : zero4;
        split_bf16x8(b0, b1, bh[j], bl[j]);
    }
    const float sc = F32 ? lo.scale : (float)(__bf16)lo.scale;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
        const float* tp = ts + (16 * i + col) * lo.rank + r0;
        const float4 t0 = r0 < lo.rank ? *reinterpret_cast<const float4*>(tp) : zero4;
        const float4 t1 = r0 + 4 < lo.rank ? *reinterpret_cast<const float4*>(tp + 4) : zero4;
        bf16x8 th, tl;
        split_bf16x8(t0, t1, th, tl);
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            f32x4 d = mfma16x16x32(th, bh[j], zero);
            d = mfma16x16x32(th, bl[j], d);
            d = mfma16x16x32(tl, bh[j], d);
            const int n = (rb0 + j) * 16 + col;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int mr = row0 + 16 * i + 4 * kq + e;
                if (mr < m_rows && n < n_rows) {
                    const long o = (long)mr * n_rows + n;
                    if constexpr (F32) {
                        const float delta = d[e] * lo.scale;
                        static_cast<float*>(y)[o] = acc[i][j][e] + delta;
                    } else {
                        const float base = (float)(__bf16)acc[i][j][e];
                        const float delta = (float)(__bf16)(d[e] * sc);
                        static_cast<uint16_t*>(y)[o] = f32_to_bf16(base + delta);
                    }
                }
            }
        }
    }
}

// LDS rings (declared per instantiation inside the kernel, sized by its tile).
// x: three slots of one group each (group g in slot g % 3; the loads for g+2 are in
// flight while g is multiplied; two slots, g % 2, for the one-pass 8-bit form on
// 256-row tiles).  Weights: two slots of one group pair each (pair p
// in slot p % 2, loaded with the x of its first group), holding the tiled words of
// the workgroup's row blocks [row block][lane] followed by their scale/bias words
// [row block][row] as uint2.  Every load is a 16-byte-per-lane DMA: 4-byte LDS DMAs
// cost the load pipe about twice the cycles for a quarter of the bytes.  Each slot is
// its own object so the compiler can tell a DMA into one slot from reads of another
// (a shared array would make it wait for every DMA before every read); it tells apart
// at most eight such objects.

// FORM: 0 the bf16 form; 1 the fp16 form (x16 from the pre-pass, B = s' (q - 8));
// 2 an 8-bit two-plane handle in one pass over K (x16 from the pre-pass, B = 1024 + q
// from the two planes' words, the per-group scale step of the bf16 form).
template <int OUT, int BM, int BN, int FORM = 0>
__global__ __launch_bounds__(BN * 2) void gemm_kernel(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                                                   const uint16_t* __restrict__ x, const uint4* __restrict__ xaug,
                                                   void* __restrict__ y, int m_rows, int n_rows, int kx, int groups,
                                                   int gpairs, int mtiles, int ntiles, int octets, uint32_t rec_bytes,
                                                   int g_split, long split_stride, int n_out,
                                                   const uint16_t* __restrict__ gelu_table, LoraEpilogue lora,
                                                   const int* __restrict__ rowexp, float s_pow, int lo_pairs) {
    // BN / 32 waves of BM x 32: BM = 256; BM = 128 (more workgroups for small M
    // without splitting K); BM = 64 (fewest K splits for narrow outputs).  FORM 1 and 2:
    // x is x16, rowexp from the pre-pass; FORM 1: s_pow = 2^p of the handle; FORM 2:
    // groups and pairs count the original K (the high plane), the low plane's pair p
    // is record lo_pairs + p.
    static_assert(BM == 256 || BM == 128 || BM == 64, "tile rows");
    static_assert(BN == 256 || BN == 128, "tile columns");
    constexpr bool F16 = FORM == 1;
    constexpr bool kQ8 = FORM == 2;
    static_assert(!F16 || BM == 256, "the fp16 form takes its group sums from the pre-pass");
    static_assert(!kQ8 || BM >= 128, "one-pass 8-bit: 128- and 256-row tiles");
    // x ring slots: three (a group's x loaded two steps ahead), or two (one step ahead)
    // where two planes' words per weight slot leave no room for a third 32 KiB slot
    // (one-pass 8-bit at 256 rows: 156 KiB against 188)
    constexpr int kXSlots = (kQ8 && BM == 256) ? 2 : 3;
    constexpr int kWaves = BN / kWN;              // side by side along N
    constexpr int kRB = BN / 16;                  // 16-row weight blocks per workgroup tile
    constexpr int kXChunks = BM * 8;              // 16-byte chunks of one x group tile (BM rows x 64 bf16)
    constexpr int kWPair = kRB * 64;              // uint4: tiled words of the pair (of one plane)
    constexpr int kWS = kQ8 ? 2 * kWPair : kWPair;  // uint4: a slot's words (both planes for FORM 2)
    constexpr int kSPair = kRB * 16 / 2;          // uint4: scale/bias words of the pair
    constexpr int kXaA = BM / 16 * 64;            // uint4: the bias A operands of the tile's rows
    constexpr int kMT = BM / 16;                  // 16x16 tiles per wave along M
    constexpr int kXParts = BM * 8 / (64 * kWaves);  // 16-byte x loads per wave per group
    // X_g summed in the kernel (64 and 128 rows), or read from xaug (256 rows, and every
    // tile of the pre-pass forms)
    constexpr bool kXIn = BM < 256 && FORM == 0;
    // in the kernel: row tiles whose X_g a wave sums, tiles wave + 8t (BM = 64: waves
    // 0-3 one each, the rest none)
    constexpr int kXTiles = kXIn ? (kMT + kWaves - 1) / kWaves : 0;
    // from xaug: 16-byte loads of bias A operands per wave per octet
    constexpr int kXaParts = BM / 16 / kWaves;
    constexpr int kSWaves = kRB / 8;              // waves that load a pair's scale words (1 KiB each)
    constexpr int kTW = kMT * kNT >= 12 ? 9 : 5;  // product-stream tile after which a pair's weights are issued
    static_assert(kRB == 2 * kWaves, "two row blocks of tiled words per wave per pair");
    static_assert(kXParts >= 1 && (kXIn ? kMT <= kXTiles * kWaves : kXaParts * kWaves == kMT),
                  "every wave loads x; every row tile's X_g is summed or loaded");
    __shared__ uint4 g_xs0[kXChunks];             // x group tiles (BM rows x 64: 16 or 32 KiB)
    __shared__ uint4 g_xs1[kXChunks];
    __shared__ uint4 g_xs2[kXSlots == 3 ? kXChunks : 1];
    __shared__ uint4 g_wp0[kWS + kSPair];         // a pair's weights: 9 or 18 KiB (34 for FORM 2)
    __shared__ uint4 g_wp1[kWS + kSPair];
    // one octet's bias operands: A side for the tile's rows [m16][lane] (written by the
    // waves, or DMA from xaug), then the scale/bias words as uint2 [row block][pair][column]
    // (DMA)
    __shared__ uint4 g_xab[kXaA + kRB * 4 * 16 / 2];
    int mt, nt;
    tile_of((int)blockIdx.x, (int)gridDim.x, mtiles, ntiles, mt, nt);
    // split of K: groups [g_begin, g_end), whole octets; with several splits each
    // writes fp32 partial sums to its own [M, N] plane of y
    // (g_split is a whole number of octets; masked so the compiler knows g_begin % 8 == 0
    // and with it the parity of every step below: no run-time selects or branches there)
    const int g_begin = (int)blockIdx.y * (g_split & ~7);
    const int g_end = groups - g_begin < g_split ? groups : g_begin + g_split;
    const int p_end = (g_end + 1) >> 1;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int rbw = nt * kRB;  // first 16-row weight block of the workgroup
    const int nblocks = (n_rows + 15) / 16;

    // sized to the buffers (<= 2^31 bytes, checked by the host) so that kOutOfRange is
    // outside every range and reads as zero
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)kx * 2u);
    const __amdgpu_buffer_rsrc_t trs = make_rsrc(tiles, rec_bytes);
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb, rec_bytes - kRecSbBytes);
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(xaug, kXIn ? 0u : (uint32_t)(mtiles * (BM / 16) * octets) * 1024u);

    // DMA issue.  Per lane, the offsets are fixed for the whole K loop (rows past M and
    // row blocks past N at kOutOfRange) and computed once here; the step moves them by
    // a scalar offset (group x 128 bytes of x, pair x one record of tiled and of scale
    // words), which stays inside the buffer for every in-range lane.  Past the
    // last group or pair the resource is swapped for an empty one: zeros, into slots
    // nobody reads again.  Branch-free, so they can sit anywhere in the product stream.
    const __amdgpu_buffer_rsrc_t zrs = make_rsrc(x, 0u);
    uint32_t xv[kXParts];  // x of a group, part u: 16-byte chunk q of the BM x 64 tile, row r,
                           // chunk c of the row, stored at position c ^ ((r >> 1) & 7) of its
                           // LDS row (swizzle: conflict-free MFMA operand reads)
#pragma unroll
    for (int u = 0; u < kXParts; ++u) {
        const int q = (kWaves * u + wave) * 64 + lane;
        const int r = q >> 3;
        const int c = (q & 7) ^ ((r >> 1) & 7);
        const int row = mt * BM + r;
        xv[u] = row < m_rows ? ((uint32_t)row * (uint32_t)kx + (uint32_t)(8 * c)) * 2u : kOutOfRange;
    }
    uint32_t wv[2];  // tiled words of a pair, part t: row block 2w + t, one 16-byte word per lane
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int rb = rbw + 2 * wave + t;
        wv[t] = rb < nblocks ? (uint32_t)rb * (uint32_t)gpairs * kRecBytes + (uint32_t)lane * 16u : kOutOfRange;
    }
    uint32_t sv;  // scale words of a pair (waves w < kSWaves): row block 8w + l/8, chunk l%8 of its 128 bytes
    {
        const int rb = rbw + 8 * wave + (lane >> 3);
        sv = rb < nblocks ? (uint32_t)rb * (uint32_t)gpairs * kRecBytes + (uint32_t)(lane & 7) * 16u : kOutOfRange;
    }
    // x rows are kx long: group g >= kx / 64 (the low plane of a two-plane handle) reads
    // group g - kx / 64 of x (a scalar select)
    const int gx = kx >> 6;
    auto dma_x = [&](int g, int part, uint4* xdst) {
        dma16(g < g_end ? xrs : zrs, xdst + (kWaves * part + wave) * 64, xv[part],
              (uint32_t)(g >= gx ? g - gx : g) * 128u);
    };
    auto dma_w = [&](int p, int part, uint4* wdst) {
        dma16(p < p_end ? trs : zrs, wdst + (2 * wave + part) * 64, wv[part], (uint32_t)p * kRecBytes);
        if constexpr (kQ8)  // the low plane's words of the same groups
            dma16(p < p_end ? trs : zrs, wdst + kWPair + (2 * wave + part) * 64, wv[part],
                  (uint32_t)(lo_pairs + p) * kRecBytes);
    };
    auto dma_s = [&](int p, uint4* wdst) {
        dma16(p < p_end ? srs : zrs, wdst + kWS + 64 * wave, sv, (uint32_t)p * kRecBytes);
    };
    // bias operands of octet o: from xaug (256 rows) the A side, kXaParts 16-byte loads;
    // the scale/bias words of its four group pairs for row blocks 2w, 2w+1 (lane l: row
    // block 2w + l/32, pair 4o + (l%32)/8, 16-byte chunk l%8 of that record's 128 bytes
    // of words)
    auto dma_xa = [&](int o) {
        int ln = threadIdx.x & 63;
        asm volatile("" : "+v"(ln));
        if constexpr (!kXIn) {
#pragma unroll
            for (int u = 0; u < kXaParts; ++u) {
                const int m16 = kXaParts * wave + u;
                dma16(ars, g_xab + m16 * 64, (uint32_t)lane * 16u, (uint32_t)(((mt * (BM / 16) + m16) * octets + o) * 1024));
            }
        }
        const int rb = rbw + 2 * wave + (ln >> 5);
        const int chunk = ln & 31;
        const bool ok = (rb < nblocks) & (4 * o + (chunk >> 3) < (kQ8 ? lo_pairs : gpairs));
        const uint32_t raw = ((uint32_t)rb * (uint32_t)gpairs + 4u * (uint32_t)o + (uint32_t)(chunk >> 3)) * kRecBytes +
                             (uint32_t)(chunk & 7) * 16u;
        dma16(srs, g_xab + (kXaA + wave * 64), ok ? raw : kOutOfRange);
    };

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const bf16x8 ones = __builtin_bit_cast(bf16x8, make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u));
    // X_g of row 16 (wave + 8t) + col for the lane's two groups of the octet (2kq, 2kq + 1)
    float xk[kXTiles > 0 ? kXTiles : 1][2];
    f32x4 xsum[kXTiles > 0 ? kXTiles : 1];  // the current group's sums: every element X_g of row col
#pragma unroll
    for (int t = 0; t < kXTiles; ++t) {
        xk[t][0] = xk[t][1] = 0.0f;
        xsum[t] = zero;
    }
    f32x4 acc[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int j = 0; j < kNT; ++j) acc[i][j] = zero;

    // one 64-wide group from LDS slots
    // hook(t) runs after the products of tile t are issued: the next group's DMA
    // instructions are spread through the product stream that way, so the CU's
    // address unit takes them while the matrix cores work (issued in one burst, all
    // eight waves would stall on it together)
    auto compute = [&](const uint4* xs, const uint4* wp, int gpar, auto&& hook) {
        // The slot arrays sit above the 64 KiB reach of a ds_read immediate offset, so
        // every (slot, constant) address would become its own register, hoisted out of
        // the loop for every slot.  An opaque lane index keeps them per step.
        int ln = threadIdx.x & 63;
        asm volatile("" : "+v"(ln));
        const int lcol = ln & 15, lkq = ln >> 4;
        const uint2* sbl = reinterpret_cast<const uint2*>(wp + kWS);
        uint2 tw[kNT];      // this group's two tiled words of each row block
        uint2 tl[kNT];      // FORM 2: the low plane's words of the same groups
        uint32_t swv[kNT];  // and its scale/bias word
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int rbl = wave * kNT + j;
            tw[j] = reinterpret_cast<const uint2*>(wp + rbl * 64 + ln)[gpar];
            if constexpr (kQ8) tl[j] = reinterpret_cast<const uint2*>(wp + kWPair + rbl * 64 + ln)[gpar];
            swv[j] = reinterpret_cast<const uint32_t*>(sbl + rbl * 16 + lcol)[gpar];
        }
        auto a_frag = [&](int i, int h) {
            const int r = 16 * i + lcol;
            return __builtin_bit_cast(bf16x8, xs[r * 8 + ((4 * h + lkq) ^ ((r >> 1) & 7))]);
        };
        // X_g of the wave's row tiles: their x fragments as the B operand
        // (B[k][n] = x[16i + n][k]) against ones, so every output of column n is the sum
        // of row n's 64 values.  Read again here rather than taken from the product
        // stream, which would need a branch per row tile.
        if (kXIn && (kMT % kWaves == 0 || wave < kMT)) {
#pragma unroll
            for (int t = 0; t < kXTiles; ++t) {
                const bf16x8 b0 = a_frag(wave + kWaves * t, 0), b1 = a_frag(wave + kWaves * t, 1);
                xsum[t] = mfma16x16x32(ones, b0, zero);
                xsum[t] = mfma16x16x32(ones, b1, xsum[t]);
            }
        }
        if constexpr (F16) {
            // The fp16 form: each tile's two products accumulate straight into its
            // outputs; row 0 expands each row block's words (s' (q - 8)) just before
            // its first products, and the next row's A operands are read a row ahead.
            f16x8 bq[kNT][2];
            bf16x8 a0 = a_frag(0, 0), a1 = a_frag(0, 1), n0, n1;
#pragma unroll
            for (int t = 0; t < kMT * kNT; ++t) {
                const int i = t / kNT, j = t % kNT;
                if (i == 0) {
                    const _Float16 sh = (_Float16)(bf16_lo(swv[j]) * s_pow);
                    const f16x2 s2 = {sh, sh};
                    bq[j][0] = expand_word_f16(tw[j].x, s2);
                    bq[j][1] = expand_word_f16(tw[j].y, s2);
                }
                if (j == 0 && i + 1 < kMT) {
                    n0 = a_frag(i + 1, 0);
                    n1 = a_frag(i + 1, 1);
                }
                acc[i][j] = mfma16x16x32(__builtin_bit_cast(f16x8, a0), bq[j][0], acc[i][j]);
                acc[i][j] = mfma16x16x32(__builtin_bit_cast(f16x8, a1), bq[j][1], acc[i][j]);
                if (j == kNT - 1) {
                    a0 = n0;
                    a1 = n1;
                }
                hook(t);
                __builtin_amdgcn_sched_barrier(0);
            }
            return;
        }
        // The wave's 32 tiles in one stream, software-pipelined and kept in this order
        // (a scheduling fence after each tile): tile t's two products, then tile t-3's
        // scale FMAs, which do not wait for them; row 0 expands each row block's words
        // just before its first products, and the next row's A operands are read one
        // row ahead.  Left to itself the compiler expands all words first and then
        // issues long runs of products with no VALU work beside them.  FORM 2 runs the
        // same stream on fp16 operands: x16 against 1024 + q, scaled by s per group (the
        // high plane's word holds 16 s).
        constexpr int kTiles = kMT * kNT;
        constexpr int kLag = 3;
        typename std::conditional<kQ8, f16x8, bf16x8>::type bq[kNT][2];
        float s16[kNT];
        f32x4 p[kLag + 1];
        bf16x8 a0 = a_frag(0, 0), a1 = a_frag(0, 1), n0, n1;
#pragma unroll
        for (int t = 0; t < kTiles + kLag; ++t) {
            if (t < kTiles) {
                const int i = t / kNT, j = t % kNT;
                if (i == 0) {
                    if constexpr (kQ8) {
                        bq[j][0] = expand_word_q8(tw[j].x, tl[j].x);
                        bq[j][1] = expand_word_q8(tw[j].y, tl[j].y);
                        s16[j] = bf16_lo(swv[j]) * 0.0625f;
                    } else {
                        bq[j][0] = expand_word(tw[j].x);
                        bq[j][1] = expand_word(tw[j].y);
                        s16[j] = bf16_lo(swv[j]) * 16.0f;
                    }
                }
                if (j == 0 && i + 1 < kMT) {
                    n0 = a_frag(i + 1, 0);
                    n1 = a_frag(i + 1, 1);
                }
                if constexpr (kQ8) {
                    p[t % (kLag + 1)] = mfma16x16x32(__builtin_bit_cast(f16x8, a0), bq[j][0], zero);
                    p[t % (kLag + 1)] = mfma16x16x32(__builtin_bit_cast(f16x8, a1), bq[j][1], p[t % (kLag + 1)]);
                } else {
                    p[t % (kLag + 1)] = mfma16x16x32(a0, bq[j][0], zero);
                    p[t % (kLag + 1)] = mfma16x16x32(a1, bq[j][1], p[t % (kLag + 1)]);
                }
                if (j == kNT - 1) {
                    a0 = n0;
                    a1 = n1;
                }
                hook(t);
            }
            if (t >= kLag) {
                const int u = t - kLag;
                const int i = u / kNT, j = u % kNT;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[i][j][e] = __builtin_fmaf(s16[j], p[u % (kLag + 1)][e], acc[i][j][e]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // bias term of the octet: A operands and scale/bias words from g_xab
    auto bias = [&]() {
        bf16x8 bb[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) bb[j] = bias_operand(reinterpret_cast<const uint2*>(g_xab + kXaA)[((wave * kNT + j) * 4 + kq) * 16 + col]);
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            const bf16x8 aa = __builtin_bit_cast(bf16x8, g_xab[i * 64 + lane]);
#pragma unroll
            for (int j = 0; j < kNT; ++j) acc[i][j] = mfma16x16x32(aa, bb[j], acc[i][j]);
        }
    };

    // Step g: (0) at g = 8o + 8, write the A operands of octet o (the slot's last
    // reads, octet o - 1's bias term, were followed by seven barriers); (1) wait until
    // this wave's loads for group g (issued during step g-2: x of g and, for even g,
    // the pair g/2) are done, leaving in flight only the loads of step g-1 (its x, for
    // even g-1 its pair, and the bias words it may have issued first), and its LDS
    // writes have landed; (2) barrier: everyone's data for g is in LDS and everyone is
    // done with the slots refilled next; (3) at g = 8o + 8, the bias term of octet o
    // (its scale/bias words were loaded at step 8o + 1 and have been waited for
    // since); at g = 8o + 1, the scale/bias words of octet o (the barrier above
    // follows the last read of the previous octet's); (4) multiply, with the loads for
    // group g+2 (and pair (g+2)/2) spread through the products, and keep the lane's
    // X_g.  Every step issues the same loads (past the end they read zeros), so the
    // counts are fixed.  With a two-slot x ring the x of g comes from step g-1 (issued
    // in its product stream before the pair's words), so (1) leaves only step g-1's
    // pair words in flight, and (4) loads the x of g+1.
    auto issues_xa = [&](int g) { return (g & 7) == 1 && g > g_begin + 1; };
    auto issued = [&](int g) {  // loads this wave issues at step g
        return kXParts + ((g & 1) == 0 ? (kQ8 ? 4 : 2) + (wave < kSWaves ? 1 : 0) : 0) +
               (issues_xa(g) ? 1 + (kXIn ? 0 : kXaParts) : 0);
    };
    // the octet's A operands of the wave's row tiles into the bias slot; X_g restarts.
    // (At the top of a step, before its barrier: written at the end of one, inlined in
    // every step of the unrolled loop, it cost 40-50 more VGPRs.)
    auto write_xa = [&]() {
#pragma unroll
        for (int t = 0; t < kXTiles; ++t) {
            if (kMT % kWaves == 0 || wave + kWaves * t < kMT) g_xab[(wave + kWaves * t) * 64 + lane] = bias_a_operand(xk[t][0], xk[t][1]);
            xk[t][0] = xk[t][1] = 0.0f;
        }
    };
    auto step = [&](int g, const uint4* xs, const uint4* wp, uint4* xs2, uint4* wp2) {
        if (kXIn && (g & 7) == 0 && g > g_begin) write_xa();
        if (g == g_begin) {
            wait_vm_lds<0>();
        } else {
            // three slots: the loads of step g - 1 may stay in flight; two: only those it
            // issued after its x loads (the next pair's words, after product tile kTW)
            const int pending = kXSlots == 3 ? issued(g - 1) : ((g - 1) & 1) == 0 ? (kQ8 ? 4 : 2) : 0;
            switch (pending) {
                case 0: wait_vm_lds<0>(); break;
                case 1: wait_vm_lds<1>(); break;
                case 2: wait_vm_lds<2>(); break;
                case 3: wait_vm_lds<3>(); break;
                case 4: wait_vm_lds<4>(); break;
                case 5: wait_vm_lds<5>(); break;
                case 6: wait_vm_lds<6>(); break;
                case 7: wait_vm_lds<7>(); break;
                case 8: wait_vm_lds<8>(); break;
                case 9: wait_vm_lds<9>(); break;
                case 10: wait_vm_lds<10>(); break;
                case 11: wait_vm_lds<11>(); break;
                default: wait_vm_lds<0>(); break;  // (not reached) safe fallback
            }
        }
        lds_barrier();
        if ((g & 7) == 0 && g > g_begin) bias();
        if (issues_xa(g)) dma_xa(g >> 3);
        // the pair's scale words (waves 0, 1), issued here rather than inside the
        // product stream, which then has no branch
        if ((g & 1) == 0 && wave < kSWaves) dma_s((g + 2) >> 1, wp2);
        const bool pair = (g & 1) == 0;
        compute(xs, wp, g & 1, [&](int t) {
            if ((t & 1) && (t >> 1) < kXParts) dma_x(g + kXSlots - 1, t >> 1, xs2);
            // the pair's two weight loads after tiles kTW and kTW + 2 (inside the stream
            // of kMT x kNT tiles: 8 of them for 64-row tiles)
            if (pair && (t == kTW || t == kTW + 2)) dma_w((g + 2) >> 1, (t - kTW) >> 1, wp2);
        });
        // lane (col, kq) keeps X_g of groups 2kq and 2kq + 1 of the octet
        const bool mine = kq == ((g & 7) >> 1);
#pragma unroll
        for (int t = 0; t < kXTiles; ++t) xk[t][g & 1] = mine ? xsum[t][0] : xk[t][g & 1];
    };

    // prologue: x of the split's first two groups, its first pair, bias operands of its
    // first octet
#pragma unroll
    for (int part = 0; part < kXParts; ++part) {
        dma_x(g_begin, part, g_xs0);
        if constexpr (kXSlots == 3) dma_x(g_begin + 1, part, g_xs1);
    }
    dma_w(g_begin >> 1, 0, g_wp0);
    dma_w(g_begin >> 1, 1, g_wp0);
    if (wave < kSWaves) dma_s(g_begin >> 1, g_wp0);
    dma_xa(g_begin >> 3);
    wait_vm<0>();

    // twelve steps per iteration: the x ring turns every 3 groups, the pair ring every 4
    if constexpr (kXSlots == 2) {
        // the x ring turns every 2 groups, the pair ring every 4; twelve steps per
        // iteration as below (a four-step body spilled: 256 VGPRs and scratch, against
        // 200 with twelve)
        for (int g = g_begin; g < g_end; g += 12) {
            step(g, g_xs0, g_wp0, g_xs1, g_wp1);
            if (g + 1 < g_end) step(g + 1, g_xs1, g_wp0, g_xs0, g_wp1);
            if (g + 2 < g_end) step(g + 2, g_xs0, g_wp1, g_xs1, g_wp0);
            if (g + 3 < g_end) step(g + 3, g_xs1, g_wp1, g_xs0, g_wp0);
            if (g + 4 < g_end) step(g + 4, g_xs0, g_wp0, g_xs1, g_wp1);
            if (g + 5 < g_end) step(g + 5, g_xs1, g_wp0, g_xs0, g_wp1);
            if (g + 6 < g_end) step(g + 6, g_xs0, g_wp1, g_xs1, g_wp0);
            if (g + 7 < g_end) step(g + 7, g_xs1, g_wp1, g_xs0, g_wp0);
            if (g + 8 < g_end) step(g + 8, g_xs0, g_wp0, g_xs1, g_wp1);
            if (g + 9 < g_end) step(g + 9, g_xs1, g_wp0, g_xs0, g_wp1);
            if (g + 10 < g_end) step(g + 10, g_xs0, g_wp1, g_xs1, g_wp0);
            if (g + 11 < g_end) step(g + 11, g_xs1, g_wp1, g_xs0, g_wp0);
        }
    } else {
        for (int g = g_begin; g < g_end; g += 12) {
            step(g, g_xs0, g_wp0, g_xs2, g_wp1);
            if (g + 1 < g_end) step(g + 1, g_xs1, g_wp0, g_xs0, g_wp1);
            if (g + 2 < g_end) step(g + 2, g_xs2, g_wp1, g_xs1, g_wp0);
            if (g + 3 < g_end) step(g + 3, g_xs0, g_wp1, g_xs2, g_wp0);
            if (g + 4 < g_end) step(g + 4, g_xs1, g_wp0, g_xs0, g_wp1);
            if (g + 5 < g_end) step(g + 5, g_xs2, g_wp0, g_xs1, g_wp1);
            if (g + 6 < g_end) step(g + 6, g_xs0, g_wp1, g_xs2, g_wp0);
            if (g + 7 < g_end) step(g + 7, g_xs1, g_wp1, g_xs0, g_wp0);
            if (g + 8 < g_end) step(g + 8, g_xs2, g_wp0, g_xs1, g_wp1);
            if (g + 9 < g_end) step(g + 9, g_xs0, g_wp0, g_xs2, g_wp1);
            if (g + 10 < g_end) step(g + 10, g_xs1, g_wp1, g_xs0, g_wp0);
            if (g + 11 < g_end) step(g + 11, g_xs2, g_wp1, g_xs1, g_wp0);
        }
    }
    // the last octet's bias term.  Its scale/bias words were loaded at step 8o + 1,
    // except for a last octet of one group (no such step): then they are loaded here;
    // its A operands are written here.  Both once every wave is past the previous
    // octet's bias term (which a last octet's first step applies).  The drain also
    // lands the zero-reading loads past the last group before the workgroup ends.
    {
        const int o = (g_end - 1) >> 3;
        wait_vm_lds<0>();
        lds_barrier();
        if (o > (g_begin >> 3) && 8 * o + 1 >= g_end) dma_xa(o);
        if constexpr (kXIn) write_xa();
        wait_vm_lds<0>();
        lds_barrier();
        bias();
    }
    if constexpr (F16 || kQ8) {
        // the pre-pass forms' sums are y 2^(k + p): rows 4kq + e of each row tile scaled back
        // (exact: a power of two).  The row index is opaque here, so the exponent loads
        // stay after the main loop (hoisted ahead of it, 64 values would stay live
        // through it and spill).
        int mrow = mt * BM + 4 * kq;
        asm volatile("" : "+v"(mrow));
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            const int m0 = mrow + 16 * i;
            int re[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) re[e] = m0 + e < m_rows ? rowexp[m0 + e] : 0;
#pragma unroll
            for (int j = 0; j < kNT; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][e] = __builtin_amdgcn_ldexpf(acc[i][j][e], -re[e]);
            // one row tile at a time (all 64 loads hoisted ahead would spill)
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // store: lane holds rows 4*kq + e of column col of each 16x16 tile.  The GeGLU
    // store takes its lane coordinates afresh (mbcnt), so nothing lane-dependent of
    // its own stays live across the main loop (some 200 VGPRs in the 256-row tile).
    const int slane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));

    if constexpr (OUT == kOutLoraBf16 || OUT == kOutLoraF32) {
        // t of the tile's rows into the x ring's first slot, free now
        float* ts = reinterpret_cast<float*>(g_xs0);
        wait_lds();  // this wave's operand reads have returned
        lds_barrier();
        lora_stage_t<BM>(lora, ts, mt * BM, m_rows, 64 * kWaves);
        lora_store<OUT == kOutLoraF32>(acc, lora, ts, y, mt * BM, rbw + wave * kNT, m_rows, n_rows, slane);
        return;
    }

    // bf16 GeGLU: the gelu table (5.5 KiB) into the x ring's first slot, free now
    const uint16_t* gtab = reinterpret_cast<const uint16_t*>(g_xs0);
    if constexpr (OUT == kOutGegluBf16) {
        constexpr int kTabChunks = kGeluTable * 2 / 16;
        static_assert(kTabChunks <= kXChunks, "the table fits one x slot");
        wait_lds();  // this wave's operand reads have returned
        lds_barrier();
        for (int t = wave * 64 + slane; t < kTabChunks; t += 64 * kWaves)
            g_xs0[t] = reinterpret_cast<const uint4*>(gelu_table)[t];
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int rb = rbw + wave * kNT + j;
            if constexpr (OUT == kOutGegluBf16) {  // rows e and e + 1 share one GeGLU pass
                // all values first, stores after the loop: with no store between them
                // the LDS table reads are issued together rather than waited for one by one
                acc[i][j][0] = geglu2(OUT, slane & 15, acc[i][j][0], acc[i][j][1], gtab);
                acc[i][j][2] = geglu2(OUT, slane & 15, acc[i][j][2], acc[i][j][3], gtab);
                continue;
            }
            if constexpr (OUT == kOutGegluF32) {  // no memory reads: value and store together
                const int c = slane & 15;
                const int m = mt * BM + 16 * i + 4 * (slane >> 4);
                const int hn = geglu2_col(c, rb);
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const float h = geglu2(OUT, c, acc[i][j][e], acc[i][j][e + 1], gtab);
                    const int mr = geglu2_row(c, m + e, m + e + 1);
                    if (mr < m_rows && hn < n_out) static_cast<float*>(y)[(long)mr * n_out + hn] = h;
                }
                continue;
            }
            const int m = mt * BM + 16 * i + 4 * kq;
            {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (OUT == kOutF32) {  // fp32 output, or this split's partial plane
                        const int n = rb * 16 + col;
                        if (m + e < m_rows && n < n_rows)
                            static_cast<float*>(y)[(long)blockIdx.y * split_stride + (long)(m + e) * n_rows + n] =
                                acc[i][j][e];
                    } else {
                        const OutParams op{y, nullptr, OUT, n_out, 0, 0.0f};
                        store_out<false>(op, m + e, m_rows, rb, col, n_rows, acc[i][j][e]);
                    }
                }
            }
        }
    }
    if constexpr (OUT == kOutGegluBf16) {
        const int c = slane & 15;
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
#pragma unroll
            for (int j = 0; j < kNT; ++j) {
                const int m = mt * BM + 16 * i + 4 * (slane >> 4);
                const int hn = geglu2_col(c, rbw + wave * kNT + j);
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const int mr = geglu2_row(c, m + e, m + e + 1);
                    if (mr < m_rows && hn < n_out) static_cast<uint16_t*>(y)[(long)mr * n_out + hn] = f32_to_bf16(acc[i][j][e]);
                }
            }
        }
    }
}

// y = sum over splits of the fp32 partial planes, in split order (deterministic)
template <bool F32OUT>
__global__ void split_reduce_kernel(const float* __restrict__ part, void* __restrict__ y, long elems, int splits) {
    const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= elems) return;
    if (i + 4 <= elems) {
        f32x4 v = *reinterpret_cast<const f32x4*>(part + i);
        for (int s = 1; s < splits; ++s) {
            const f32x4 w = *reinterpret_cast<const f32x4*>(part + (long)s * elems + i);
            v[0] += w[0];
            v[1] += w[1];
            v[2] += w[2];
            v[3] += w[3];
        }
        if (F32OUT) {
            float* yf = static_cast<float*>(y) + i;
            if ((reinterpret_cast<uintptr_t>(yf) & 15) == 0) {
                *reinterpret_cast<f32x4*>(yf) = v;
            } else {
                yf[0] = v[0];
                yf[1] = v[1];
                yf[2] = v[2];
                yf[3] = v[3];
            }
        } else {
            uint16_t* yb = static_cast<uint16_t*>(y) + i;
            const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
            const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
            if ((reinterpret_cast<uintptr_t>(yb) & 7) == 0) {
                *reinterpret_cast<uint2*>(yb) = make_uint2(lo, hi);
            } else {
                yb[0] = (uint16_t)lo;
                yb[1] = (uint16_t)(lo >> 16);
                yb[2] = (uint16_t)hi;
                yb[3] = (uint16_t)(hi >> 16);
            }
        }
    } else {
        for (long j = i; j < elems; ++j) {
            float v = part[j];
            for (int s = 1; s < splits; ++s) v += part[(long)s * elems + j];
            if (F32OUT)
                static_cast<float*>(y)[j] = v;
            else
                static_cast<uint16_t*>(y)[j] = f32_to_bf16(v);
        }
    }
}

// gelu_bf16 of the table's bf16 patterns (the table the bf16 GeGLU epilogue reads)
__global__ void gelu_table_kernel(uint16_t* __restrict__ table) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < kGeluTable) table[i] = f32_to_bf16(gelu_bf16(__uint_as_float(gelu_table_pattern(i) << 16)));
}

// h = GeGLU of the summed gate|up partial planes, in split order (deterministic).  One
// thread per output h[m, hn]: gate and up are columns 16*(hn/8) + hn%8 and that + 8.
template <int OUT>
__global__ void split_geglu_kernel(const float* __restrict__ part, void* __restrict__ h, int m_rows, int n_rows,
                                   int n_out, long elems, int splits) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)m_rows * n_out) return;
    const int m = (int)(i / n_out);
    const int hn = (int)(i - (long)m * n_out);
    const long o = (long)m * n_rows + (hn >> 3) * 16 + (hn & 7);
    float g = part[o], u = part[o + 8];
    for (int s = 1; s < splits; ++s) {
        g += part[(long)s * elems + o];
        u += part[(long)s * elems + o + 8];
    }
    if (OUT == kOutGegluF32)
        static_cast<float*>(h)[i] = geglu_f32(g, u);
    else
        static_cast<uint16_t*>(h)[i] = f32_to_bf16(geglu_bf16(g, u));
}

}  // namespace

// Tile shape and split of K.  For each tile shape (256, 128 or 64 rows x 256) and split
// count (whole octets per split), the cost is
//   rounds of workgroups x (groups per split x the step time + kRoundUs)
//   + for a split: kSplitUs + the partial sums' bytes / kPartialBytesPerUs
//   + for the 256-row tile: kPrePassUs (its X_g pre-pass launch),
// and the cheapest wins.  The constants are fitted to every plan measured on the eight
// prefill shapes (q, k, o, gate, down, the gate|up pair, the full-attention q and o) at
// 14 row counts from 64 to 2048, every tile at every row count: the picks average 0.7%
// and at worst 7.4% over the fastest plan of each case.  (The constants fitted to the
// kernel with the pre-pass for every tile, the 64-row tile offered up to 128 rows,
// give 3.7% and 26% on the same measurements.)
namespace {
struct TileShape {
    int bm, bn, per_cu;
    double step_us;  // one 64-wide group step of a workgroup (fitted with the constants below)
    int max_m;       // offered up to this many rows (0: any)
};
// The 64-row tile pads least and, unsplit, needs no scratch; it wins wherever it fills
// the CUs with fewer K splits.  Best plan of each tile, measured: at 64 rows the
// 128-row tile, half of it padding, is 10-26% behind (q 4096x3840 26.3 us vs 29.2, gate
// 15360x3840 30.2 vs 36.1, the gate|up pair 41.7 vs 52.7); at 2048 rows k 2048x3840
// runs 45.9 us on it unsplit against 57.7 on the 128-row tile split in two, and at 512
// rows the full-attention q 8192x3840 46.5 vs 57.6.  Step times are fitted at one
// workgroup per CU (the 64-row tile fits two, but each then runs at half the rate).
constexpr TileShape kTileShapes[] = {{256, 256, 1, 1.8, 0}, {128, 256, 1, 1.1, 0}, {64, 256, 1, 0.65, 0}};
constexpr double kRoundUs = 1.0;               // per round of workgroups: prologue, epilogue, ramp
constexpr double kSplitUs = 4.0;               // a split's reduction launch
constexpr double kPartialBytesPerUs = 4.0e6;   // partial sums written and read back
constexpr double kPrePassUs = 3.0;             // the 256-row tile's group-sum pre-pass
// the fp16 form: its group step against the bf16 form's (gate 15360x3840 at 2048 rows,
// the kernel alone, steady clock: 210-215 vs 218-223 us), and its pre-pass's extra
// time per byte of x16 (12.3 us against the group-sum pre-pass's 5.0 for 15.7 MB)
constexpr double kF16StepScale = 0.965;
constexpr double kPrepBytesPerUs = 2.15e6;
// one-pass 8-bit: its group step (over K, not 2K) against the 4-bit tile's of the
// same height (8-bit gate 15360x3840 at 2048 rows with the pre-pass: 262 us on 256-row
// tiles, 120 steps per CU: 1.16; 325 on 128-row tiles, 240 steps: 1.19)
constexpr double kQ8StepScale = 1.2;
size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }
}  // namespace

void set_f16_form(Layout& l, const int range[3]) {
    l.f16 = false;
    l.f16_p = 0;
    if (range[2] != 0 || l.kx / 64 > kPrepMaxGroups) return;
    if (range[0] < 0) {  // every scale zero
        l.f16 = true;
        return;
    }
    // the largest scale times 2^p in [2^12, 2^13); the smallest nonzero then >= 2^-14
    // when the exponents span at most 26 (subnormal scales, exponent 0, need p > 64:
    // those handles keep the bf16 form)
    const int p = 12 - (range[0] - 127);
    if (range[0] - range[1] > 26 || p > 64 || p < -64) return;
    l.f16 = true;
    l.f16_p = p;
}

hipError_t launch_scale_range(const uint2* sb, const Layout& l, int* out, hipStream_t stream) {
    const long records = (long)l.nb * l.gp;
    const long threads = records * 16;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(scale_range_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, sb, records,
                       out);
    return hipGetLastError();
}

GemmPlan plan_gemm(int m, const Layout& l, size_t max_workspace) {
    GemmPlan p;
    const long cus = device_cus();
    // one-pass 8-bit: a two-plane handle whose low plane's group pairs line up with the
    // high plane's (an even number of groups per plane)
    const bool q8_ok = l.prepass_forms && l.k == 2 * l.kx && (l.g / 2) % 2 == 0 && l.kx / 64 <= kPrepMaxGroups;
    double best = -1.0;
    for (const TileShape& ts : kTileShapes) {
        if (ts.max_m > 0 && m > ts.max_m) continue;
        const int bm = ts.bm, bn = ts.bn;
        const long tiles = (long)((m + bm - 1) / bm) * ((l.n + bn - 1) / bn);
        // form 0: the bf16 form; 1: the fp16 form (256-row tiles of handles whose scales
        // allow it); 2: one-pass 8-bit (128- and 256-row tiles)
        for (int form = 2; form >= 0; --form) {
            if ((form == 1 && !(bm == 256 && l.f16 && l.prepass_forms)) || (form == 2 && !(bm >= 128 && q8_ok)))
                continue;
            const bool pre = form != 0;
            const int groups = form == 2 ? l.g / 2 : l.g;
            const int octets = (groups + 7) / 8;
            // the X_g pre-pass (bias A operands of every 16-row block and octet) of the
            // 256-row tile and of the pre-pass forms; their x16 and row exponents
            const size_t xa = (bm == 256 || pre) ? ((size_t)m + bm - 1) / bm * (bm / 16) * octets * 1024 : 0;
            const size_t x16 = pre ? round256((size_t)m * l.kx * 2) : 0;
            const size_t rexp = pre ? round256((size_t)m * 4) : 0;
            for (int s = 1; s <= octets && s <= kMaxSplits; ++s) {
                const int per = (octets + s - 1) / s;
                const int used = (octets + per - 1) / per;  // splits that get work
                if (used != s) continue;
                const size_t part = s > 1 ? (size_t)s * m * l.n * 4 : 0;
                if (part > kMaxPartialBytes) break;
                if (xa + x16 + rexp + part > max_workspace) break;  // (more splits need more)
                const double rounds = (double)((tiles * s + cus * ts.per_cu - 1) / (cus * ts.per_cu));
                const double step = ts.step_us * (form == 1 ? kF16StepScale : form == 2 ? kQ8StepScale : 1.0);
                const double t = rounds * (per * 8 * step + kRoundUs) +
                                 (s > 1 ? kSplitUs + part / kPartialBytesPerUs : 0.0) +
                                 ((bm == 256 || pre) ? kPrePassUs + x16 / kPrepBytesPerUs : 0.0);
                if (best < 0.0 || t < best) {
                    best = t;
                    p.bm = bm;
                    p.bn = bn;
                    p.splits = s;
                    p.g_split = per * 8;
                    p.part_bytes = part;
                    p.xaug_bytes = xa;
                    p.f16 = form == 1;
                    p.q8 = form == 2;
                    p.x16_bytes = x16;
                    p.rowexp_bytes = rexp;
                }
            }
        }
    }
    return p;
}

size_t gemm_workspace_bytes(int m, const Layout& l) { return plan_gemm(m, l).total(); }

hipError_t launch_gelu_table(uint16_t* table, hipStream_t stream) {
    hipLaunchKernelGGL(gelu_table_kernel, dim3((kGeluTable + 255) / 256), dim3(256), 0, stream, table);
    return hipGetLastError();
}

bool gemm_lora_epilogue(int m, const Layout& l, int rank, size_t workspace_bytes) {
    return rank >= 4 && rank <= 32 && rank % 4 == 0 && plan_gemm(m, l, workspace_bytes).splits == 1;
}

hipError_t launch_gemm(const uint4* tiles, const uint2* sb, const uint16_t* x, void* y, int m, int out_mode,
                       int n_out, const Layout& l, void* workspace, size_t workspace_bytes,
                       const uint16_t* gelu_table, hipStream_t stream, const LoraEpilogue* lora) {
    const GemmPlan plan = plan_gemm(m, l, workspace_bytes);
    if (plan.total() > workspace_bytes) return hipErrorInvalidValue;
    const LoraEpilogue lo = lora != nullptr ? *lora : LoraEpilogue{nullptr, nullptr, 0, 0, 0.0f};
    if (lora != nullptr && (plan.splits != 1 || out_mode > kOutF32 || lo.rank % 4 != 0 || lo.rank < 4 ||
                            lo.rank > 32 || lo.slices < 1 || lo.part == nullptr || lo.b == nullptr))
        return hipErrorInvalidValue;
    // one-pass 8-bit: groups and octets of K (the high plane), the low plane from pair
    // groups / 2 of each row block's records
    const int groups = plan.q8 ? l.g / 2 : l.g;
    const int octets = (groups + 7) / 8;
    const int lo_pairs = plan.q8 ? groups / 2 : 0;
    const int mtiles = (m + plan.bm - 1) / plan.bm;
    const int ntiles = (l.n + plan.bn - 1) / plan.bn;
    // workspace: [group sums | x16 | row exponents | partial sums], each 256-byte aligned
    char* const wsb = static_cast<char*>(workspace);
    uint4* xaug = plan.xaug_bytes ? reinterpret_cast<uint4*>(wsb) : nullptr;
    const bool pre = plan.f16 || plan.q8;
    uint16_t* x16 = pre ? reinterpret_cast<uint16_t*>(wsb + plan.xaug_bytes) : nullptr;
    int* rowexp = pre ? reinterpret_cast<int*>(wsb + plan.xaug_bytes + plan.x16_bytes) : nullptr;
    float* part = reinterpret_cast<float*>(wsb + plan.xaug_bytes + plan.x16_bytes + plan.rowexp_bytes);
    if (l.rec_bytes() > kMaxBufferBytes || (size_t)m * l.kx * 2 > kMaxBufferBytes || plan.xaug_bytes > kMaxBufferBytes)
        return hipErrorInvalidValue;
    if (pre) {
        // one wave per row of the tiles
        const dim3 pg((unsigned)(mtiles * plan.bm / kPrepRows)), pb(64 * kPrepRows);
        const size_t plds = (size_t)kPrepRows * (l.kx / 64) * sizeof(float);
        if (plan.q8)
            hipLaunchKernelGGL(xprep_kernel<-64>, pg, pb, plds, stream, x, x16, xaug, rowexp, m, l.kx, groups, octets, 0);
        else
            hipLaunchKernelGGL(xprep_kernel<8>, pg, pb, plds, stream, x, x16, xaug, rowexp, m, l.kx, groups, octets,
                               l.f16_p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    } else if (plan.xaug_bytes) {
        const long units = (long)mtiles * (plan.bm / 16) * octets;  // 1 KiB blocks
        hipLaunchKernelGGL(xaug_kernel, dim3((unsigned)units), dim3(512), 0, stream, x, xaug, m, l.kx, l.g, octets);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const uint16_t* const xin = pre ? x16 : x;
    const float s_pow = plan.f16 ? __builtin_ldexpf(1.0f, l.f16_p) : 1.0f;
    const dim3 grid((unsigned)(mtiles * ntiles), (unsigned)plan.splits), block(2 * plan.bn);
    const uint32_t rec_bytes = (uint32_t)l.rec_bytes();
    const long elems = (long)m * l.n;
    // one instantiation per (output mode, tile shape, form)
#define Q4_GEMM_ARGS(YPTR, STRIDE)                                                                               \
    tiles, sb, xin, xaug, YPTR, m, l.n, l.kx, groups, l.gp, mtiles, ntiles, octets, rec_bytes, plan.g_split,      \
        STRIDE, n_out, gelu_table, lo, rowexp, s_pow, lo_pairs
#define Q4_GEMM_LAUNCH(MODE, YPTR, STRIDE)                                                                       \
    do {                                                                                                         \
        if (plan.bm == 64)                                                                                       \
            hipLaunchKernelGGL((gemm_kernel<MODE, 64, 256>), grid, block, 0, stream, Q4_GEMM_ARGS(YPTR, STRIDE));  \
        else if (plan.bm == 256 && plan.f16)                                                                     \
            hipLaunchKernelGGL((gemm_kernel<MODE, 256, 256, 1>), grid, block, 0, stream,                         \
                               Q4_GEMM_ARGS(YPTR, STRIDE));                                                      \
        else if (plan.bm == 128 && plan.q8)                                                                      \
            hipLaunchKernelGGL((gemm_kernel<MODE, 128, 256, 2>), grid, block, 0, stream,                         \
                               Q4_GEMM_ARGS(YPTR, STRIDE));                                                      \
        else if (plan.bm == 256 && plan.q8)                                                                      \
            hipLaunchKernelGGL((gemm_kernel<MODE, 256, 256, 2>), grid, block, 0, stream,                         \
                               Q4_GEMM_ARGS(YPTR, STRIDE));                                                      \
        else if (plan.bm == 256)                                                                                 \
            hipLaunchKernelGGL((gemm_kernel<MODE, 256, 256>), grid, block, 0, stream, Q4_GEMM_ARGS(YPTR, STRIDE)); \
        else                                                                                                     \
            hipLaunchKernelGGL((gemm_kernel<MODE, 128, 256>), grid, block, 0, stream, Q4_GEMM_ARGS(YPTR, STRIDE)); \
    } while (0)
    if (plan.splits > 1) {
        Q4_GEMM_LAUNCH(kOutF32, (void*)part, elems);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int rblock = 256;
        if (out_mode >= kOutGegluBf16) {
            const unsigned rgrid = (unsigned)(((long)m * n_out + rblock - 1) / rblock);
            if (out_mode == kOutGegluF32)
                hipLaunchKernelGGL((split_geglu_kernel<kOutGegluF32>), dim3(rgrid), dim3(rblock), 0, stream, part, y, m,
                                   l.n, n_out, elems, plan.splits);
            else
                hipLaunchKernelGGL((split_geglu_kernel<kOutGegluBf16>), dim3(rgrid), dim3(rblock), 0, stream, part, y, m,
                                   l.n, n_out, elems, plan.splits);
            return hipGetLastError();
        }
        const unsigned rgrid = (unsigned)(((elems + 3) / 4 + rblock - 1) / rblock);
        if (out_mode == kOutF32)
            hipLaunchKernelGGL((split_reduce_kernel<true>), dim3(rgrid), dim3(rblock), 0, stream, part, y, elems,
                               plan.splits);
        else
            hipLaunchKernelGGL((split_reduce_kernel<false>), dim3(rgrid), dim3(rblock), 0, stream, part, y, elems,
                               plan.splits);
        return hipGetLastError();
    }
    if (lora != nullptr) {
        if (out_mode == kOutF32)
            Q4_GEMM_LAUNCH(kOutLoraF32, y, 0L);
        else
            Q4_GEMM_LAUNCH(kOutLoraBf16, y, 0L);
        return hipGetLastError();
    }
    switch (out_mode) {
        case kOutF32: Q4_GEMM_LAUNCH(kOutF32, y, 0L); break;
        case kOutGegluBf16: Q4_GEMM_LAUNCH(kOutGegluBf16, y, 0L); break;
        case kOutGegluF32: Q4_GEMM_LAUNCH(kOutGegluF32, y, 0L); break;
        default: Q4_GEMM_LAUNCH(kOutBf16, y, 0L); break;
    }
#undef Q4_GEMM_LAUNCH
#undef Q4_GEMM_ARGS
    return hipGetLastError();
}

}  // namespace q4
