// Prefill-shape affine-Q4 matmul on gfx950: y[M,N] = x[M,K] . W^T for large M.
//
// Exact factored form on the matrix cores (q4_common.h):
//   y = sum_g 16*s_g * P_g + (b_g - 16*s_g) * X_g,   P_g = sum_{k in g} x*(1 + q/16)
// * P_g: two v_mfma_f32_16x16x32_bf16 per 16x16 tile per group, B operands expanded
//   from the tiled nibbles in registers (no dequantized weights anywhere), then
//   acc += 16*s * P_g on the fp32 accumulators (one VALU FMA per output per group);
// * the bias term: one extra MFMA per tile per 8 groups on an augmented K of 32,
//   A = [Xh, Xl, -16Xh, -16Xl] per group (X_g = Xh + Xl split into two bf16, from
//   xaug_kernel), B = [b, b, s, s] taken straight from the scale/bias words.
// Every product is exact; rounding is fp32 accumulation only.
//
// Tiling: a 512-thread workgroup computes a 256 (M) x 256 (N) tile as 2 x 4 waves
// of 128 x 64 (two waves per SIMD, so one's MFMA and LDS latencies are covered by
// the other's work).  Everything streams through LDS by direct-to-LDS buffer loads
// (no staging registers): per 64-wide group the x tile (rows swizzled so the MFMA
// operand reads are bank-conflict free), the group's weight words and scale words;
// the bias operands once per 8 groups.  The rings have three slots, so each load has
// two steps of arithmetic to arrive in.
#include "q4_common.h"
#include "q4_kernels.h"

namespace q4 {
namespace {

constexpr int kBM = 256;              // workgroup tile rows (M)
constexpr int kBN = 256;              // workgroup tile columns (N)
constexpr int kWaves = 8;             // 2 (M) x 4 (N) waves, two per SIMD
constexpr int kRB = kBN / 16;         // 16-row weight blocks per workgroup tile
constexpr int kWM = 128;              // wave tile rows
constexpr int kWN = 64;               // wave tile columns
constexpr int kMT = kWM / 16;         // 16x16 tiles per wave along M
constexpr int kNT = kWN / 16;         // 16x16 tiles per wave along N
constexpr int kXChunks = kBM * 8;     // 16-byte chunks of one x group tile (256 rows x 64 bf16)

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// ---------------------------------------------------------------------------
// X_g = sum of x over each 64-wide group, as the augmented-K MFMA A operand:
// xaug[m16][octet][lane] (16 B), lane (m = l%16, kq = l/16), element e ->
// group 8*octet + 2*kq + e/4, term e%4 in {Xh, Xl, -16 Xh, -16 Xl}.
// ---------------------------------------------------------------------------
__global__ void xaug_kernel(const uint16_t* __restrict__ x, uint4* __restrict__ xaug, int m_rows, int k,
                            int groups, int octets, long total) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int lane = (int)(tid & 63);
    const long t = tid >> 6;
    const int o = (int)(t % octets);
    const long mb = t / octets;
    const long m = mb * 16 + (lane & 15);
    const int kq = lane >> 4;
    uint32_t w[4];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = 8 * o + 2 * kq + gi;
        float sum = 0.f;
        if (m < m_rows && g < groups) {
            const uint4* src = reinterpret_cast<const uint4*>(x + m * k + 64 * g);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint4 v = src[c];
                sum += bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y) + bf16_lo(v.z) + bf16_hi(v.z) +
                       bf16_lo(v.w) + bf16_hi(v.w);
            }
        }
        const uint16_t xh = f32_to_bf16(sum);
        const uint16_t xl = f32_to_bf16(sum - __uint_as_float((uint32_t)xh << 16));
        const uint16_t nxh = f32_to_bf16(-16.0f * __uint_as_float((uint32_t)xh << 16));
        const uint16_t nxl = f32_to_bf16(-16.0f * __uint_as_float((uint32_t)xl << 16));
        w[2 * gi] = (uint32_t)xh | ((uint32_t)xl << 16);
        w[2 * gi + 1] = (uint32_t)nxh | ((uint32_t)nxl << 16);
    }
    xaug[tid] = make_uint4(w[0], w[1], w[2], w[3]);
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

// LDS ring buffers, three slots each (group g uses slot g % 3; the loads for g+2 are
// in flight while g is multiplied).  Each slot is its own object so the compiler
// can tell a DMA into one slot from reads of another (a shared array would make it
// wait for every DMA before every read).
__shared__ uint4 g_xs0[kXChunks];          // x group tile, 256 rows x 64 (32 KiB)
__shared__ uint4 g_xs1[kXChunks];
__shared__ uint4 g_xs2[kXChunks];
__shared__ uint32_t g_wt0[kRB * 2 * 64];   // the group's weight words: [row block][half][lane] (8 KiB)
__shared__ uint32_t g_wt1[kRB * 2 * 64];
__shared__ uint32_t g_wt2[kRB * 2 * 64];
__shared__ uint32_t g_sb0[kRB * 16];       // the group's scale/bias words: [row block][column] (1 KiB)
__shared__ uint32_t g_sb1[kRB * 16];
__shared__ uint32_t g_sb2[kRB * 16];
__shared__ uint4 g_xa[16 * 64];            // bias-MFMA A operands of the 256 rows for one octet (16 KiB)

// s_waitcnt with vmcnt(n) only (expcnt / lgkmcnt left free), n < 64
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
// the same plus lgkmcnt(0): this wave's LDS reads have returned
template <int N>
__device__ __forceinline__ void wait_vm_lds() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

template <bool F32OUT>
__global__ __launch_bounds__(512) void gemm_kernel(const uint4* __restrict__ tiles, const uint2* __restrict__ sb,
                                                   const uint16_t* __restrict__ x, const uint4* __restrict__ xaug,
                                                   void* __restrict__ y, int m_rows, int n_rows, int k, int groups,
                                                   int gpairs, int mtiles, int ntiles, int octets, uint32_t tile_bytes,
                                                   uint32_t sb_bytes) {
    int mt, nt;
    tile_of((int)blockIdx.x, (int)gridDim.x, mtiles, ntiles, mt, nt);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int wm = wave & 1;
    const int wn = wave >> 1;
    const int rbw = nt * kRB;  // first 16-row weight block of the workgroup
    const int nblocks = (n_rows + 15) / 16;

    // sized to the buffers (<= 2^31 bytes, checked by the host) so that kOutOfRange is
    // outside every range and reads as zero
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)k * 2u);
    const __amdgpu_buffer_rsrc_t trs = make_rsrc(tiles, tile_bytes);
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb, sb_bytes);
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(xaug, (uint32_t)(mtiles * 16 * octets) * 1024u);

    // ---- DMA issue, per wave and group: x 4, weight words 4, scale words 1; bias
    // operands 2 per octet ----
    uint32_t xoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int q = (8 * u + wave) * 64 + lane;  // 16-byte chunk of the 256 x 64 tile
        const int r = q >> 3;
        const int c = (q & 7) ^ ((r >> 1) & 7);  // swizzled: chunk c of row r sits at position c ^ ((r>>1)&7)
        const int row = mt * kBM + r;
        xoff[u] = row < m_rows ? (uint32_t)(row * k + 8 * c) * 2u : kOutOfRange;
    }
    auto dma = [&](int g, uint4* xdst, uint32_t* wdst, uint32_t* sdst) {
        const uint32_t gofs = (uint32_t)g * 128u;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t off = xoff[u] == kOutOfRange ? kOutOfRange : xoff[u] + gofs;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_ptr_t)(xdst + (8 * u + wave) * 64), 16, off, 0, 0, 0);
        }
        // weight words of the group: row block rbl = 2w + t, half h -> tile word 2*(g&1) + h
        const int gp = g >> 1;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int rbl = 2 * wave + t;
            const int rb = rbw + rbl;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t off =
                    rb < nblocks ? (uint32_t)((((long)rb * gpairs + gp) * 64 + lane) * 16 + (2 * (g & 1) + h) * 4)
                                 : kOutOfRange;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(trs, (lds_ptr_t)(wdst + (rbl * 2 + h) * 64), 4, off, 0, 0, 0);
            }
        }
        if (lane < 32) {  // 32 lanes x 4 B: scale words of row blocks 2w, 2w+1
            const int rbl = 2 * wave + (lane >> 4);
            const int rb = rbw + rbl;
            const uint32_t off =
                rb < nblocks ? (uint32_t)((((long)rb * gpairs + gp) * 16 + (lane & 15)) * 8 + (g & 1) * 4)
                             : kOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_ptr_t)(sdst + 32 * wave), 4, off, 0, 0, 0);
        }
    };
    auto dma_xa = [&](int o) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int m16 = 2 * wave + u;
            const uint32_t off = (uint32_t)((((long)mt * 16 + m16) * octets + o) * 1024 + lane * 16);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (lds_ptr_t)(g_xa + m16 * 64), 16, off, 0, 0, 0);
        }
    };

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int j = 0; j < kNT; ++j) acc[i][j] = zero;

    // one 64-wide group from LDS slots
    auto compute = [&](const uint4* xs, const uint32_t* wt, const uint32_t* sbl) {
        bf16x8 bq[kNT][2];
        float s16[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int rbl = wn * kNT + j;
            bq[j][0] = expand_word(wt[(rbl * 2 + 0) * 64 + lane]);
            bq[j][1] = expand_word(wt[(rbl * 2 + 1) * 64 + lane]);
            s16[j] = bf16_lo(sbl[rbl * 16 + col]) * 16.0f;
        }
        auto a_frag = [&](int i, int h) {
            const int r = wm * kWM + 16 * i + col;
            return __builtin_bit_cast(bf16x8, xs[r * 8 + ((4 * h + kq) ^ ((r >> 1) & 7))]);
        };
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            const bf16x8 a0 = a_frag(i, 0), a1 = a_frag(i, 1);
            f32x4 p[kNT];
#pragma unroll
            for (int j = 0; j < kNT; ++j) p[j] = mfma16x16x32(a0, bq[j][0], zero);
#pragma unroll
            for (int j = 0; j < kNT; ++j) p[j] = mfma16x16x32(a1, bq[j][1], p[j]);
#pragma unroll
            for (int j = 0; j < kNT; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][e] = __builtin_fmaf(s16[j], p[j][e], acc[i][j][e]);
        }
    };
    // bias term of octet o: A operands from g_xa, B from the scale words (global)
    auto bias = [&](const uint2* bw) {
        bf16x8 bb[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) bb[j] = bias_operand(bw[j]);
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            const bf16x8 aa = __builtin_bit_cast(bf16x8, g_xa[(wm * kMT + i) * 64 + lane]);
#pragma unroll
            for (int j = 0; j < kNT; ++j) acc[i][j] = mfma16x16x32(aa, bb[j], acc[i][j]);
        }
    };
    auto load_bias_words = [&](int o, uint2* bw) {
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int rb = rbw + wn * kNT + j;
            const int gp = 4 * o + kq;
            const bool ok = rb < nblocks && gp < gpairs;
            bw[j] = buffer_load8(srs, ok ? (uint32_t)(((long)rb * gpairs + gp) * 128 + col * 8) : kOutOfRange);
        }
    };

    // Step g: (1) wait until this wave's DMAs for group g (issued at step g-2 in the
    // order x, weights, scales; bias operands at the octet start) are done, leaving in
    // flight only what was issued after them; (2) barrier: everyone's data for g is in
    // LDS and everyone is done with the slot refilled next; (3) issue the DMAs for
    // group g+2 (and at octet starts the octet's bias operands); (4) multiply.
    auto issues = [&](int g) { return g + 2 < groups; };
    auto issues_xa = [&](int g) { return (g & 7) == 0 && g > 0; };
    auto step = [&](int g, const uint4* xs, const uint32_t* wt, const uint32_t* sbl, uint4* xs2, uint32_t* wt2,
                    uint32_t* sb2) {
        const int after = (g >= 2 && issues_xa(g - 2) ? 2 : 0) +
                          (g >= 1 ? (issues(g - 1) ? 9 : 0) + (issues_xa(g - 1) ? 2 : 0) : 0);
        switch (after) {
            case 0: wait_vm_lds<0>(); break;
            case 2: wait_vm_lds<2>(); break;
            case 9: wait_vm_lds<9>(); break;
            case 11: wait_vm_lds<11>(); break;
            case 13: wait_vm_lds<13>(); break;
            default: wait_vm_lds<0>(); break;  // (not reached) safe fallback
        }
        __builtin_amdgcn_s_barrier();
        const bool octet_end = (g & 7) == 7 || g == groups - 1;
        uint2 bw[kNT];
        if (octet_end) load_bias_words(g >> 3, bw);  // before this step's DMAs: waiting on it skips them
        if (issues(g)) dma(g + 2, xs2, wt2, sb2);
        if (issues_xa(g)) dma_xa(g >> 3);
        compute(xs, wt, sbl);
        if (octet_end) bias(bw);
    };

    // prologue: groups 0 and 1, bias operands of octet 0
    dma(0, g_xs0, g_wt0, g_sb0);
    if (groups > 1) dma(1, g_xs1, g_wt1, g_sb1);
    dma_xa(0);
    wait_vm<0>();

    for (int g = 0; g < groups; g += 3) {
        step(g, g_xs0, g_wt0, g_sb0, g_xs2, g_wt2, g_sb2);
        if (g + 1 < groups) step(g + 1, g_xs1, g_wt1, g_sb1, g_xs0, g_wt0, g_sb0);
        if (g + 2 < groups) step(g + 2, g_xs2, g_wt2, g_sb2, g_xs1, g_wt1, g_sb1);
    }

    // store: lane holds rows 4*kq + e of column col of each 16x16 tile
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int n = (rbw + wn * kNT + j) * 16 + col;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = mt * kBM + wm * kWM + 16 * i + 4 * kq + e;
                if (m < m_rows && n < n_rows) {
                    const long o = (long)m * n_rows + n;
                    if (F32OUT)
                        static_cast<float*>(y)[o] = acc[i][j][e];
                    else
                        static_cast<uint16_t*>(y)[o] = f32_to_bf16(acc[i][j][e]);
                }
            }
        }
    }
}

}  // namespace

size_t gemm_workspace_bytes(int m, const Layout& l) {
    const size_t m16 = ((size_t)m + kBM - 1) / kBM * (kBM / 16);
    const size_t octets = ((size_t)l.g + 7) / 8;
    return m16 * octets * 64 * 16;
}

hipError_t launch_gemm(const uint4* tiles, const uint2* sb, const uint16_t* x, void* y, int m, bool out_f32,
                       const Layout& l, void* workspace, hipStream_t stream) {
    const int octets = (l.g + 7) / 8;
    const int mtiles = (m + kBM - 1) / kBM;
    const int ntiles = (l.n + kBN - 1) / kBN;
    uint4* xaug = static_cast<uint4*>(workspace);
    {
        const long total = (long)mtiles * (kBM / 16) * octets * 64;
        const int block = 256;
        hipLaunchKernelGGL(xaug_kernel, dim3((unsigned)((total + block - 1) / block)), dim3(block), 0, stream, x, xaug, m,
                           l.k, l.g, octets, total);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const dim3 grid((unsigned)(mtiles * ntiles)), block(64 * kWaves);
    if (l.tile_bytes() > kMaxBufferBytes || l.sb_bytes() > kMaxBufferBytes ||
        (size_t)m * l.k * 2 > kMaxBufferBytes)
        return hipErrorInvalidValue;
    const uint32_t tb = (uint32_t)l.tile_bytes(), sbb = (uint32_t)l.sb_bytes();
    if (out_f32)
        hipLaunchKernelGGL((gemm_kernel<true>), grid, block, 0, stream, tiles, sb, x, xaug, y, m, l.n, l.k, l.g, l.gp,
                           mtiles, ntiles, octets, tb, sbb);
    else
        hipLaunchKernelGGL((gemm_kernel<false>), grid, block, 0, stream, tiles, sb, x, xaug, y, m, l.n, l.k, l.g, l.gp,
                           mtiles, ntiles, octets, tb, sbb);
    return hipGetLastError();
}

}  // namespace q4
