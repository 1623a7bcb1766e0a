// Host-side launchers of the gfx950 affine-Q4 kernels (internal to libgemma4_qmm).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace q4 {

// Weight records: one per (16-row block, group pair), [row block][pair], 1152 bytes
// each: the 1 KiB tile of tiled words (uint4 per lane) and then the block's 16 scale/
// bias words for the pair (uint2 per row), so a kernel streaming a row block reads one
// contiguous run.  Kernels take the record array as uint4 tiles (record t's words at
// t * kRecU4 + lane) and as uint2 sb starting kRecSbBytes into it (record t's word for
// row r at t * kRecU2 + r).
constexpr int kRecBytes = 1152;
constexpr int kRecSbBytes = 1024;
constexpr int kRecU4 = kRecBytes / 16;
constexpr int kRecU2 = kRecBytes / 8;

// Bytes from the first of n consecutive records' scale/bias words to the end of the
// last record: the size of a buffer resource over their words (0 for none, so that
// every offset reads as zero).
__host__ __device__ inline uint32_t sb_span(int n) {
    return n > 0 ? (uint32_t)n * (uint32_t)kRecBytes - (uint32_t)kRecSbBytes : 0u;
}

struct Layout {
    int n = 0;   // output features
    int k = 0;   // input features of the tiled weight (2K for two-plane 8-bit handles)
    int kx = 0;  // row length of x: k, or K = k / 2 for two-plane handles, whose kernels
                 // read column c of x' = [x | x] as column c mod K of x
    int g = 0;   // groups per row (k / 64)
    int nb = 0;  // 16-row blocks
    int gp = 0;  // group pairs (ceil(g / 2))
    // the GEMM's fp16 form applies (set when the handle is built, from its scales: every
    // nonzero scale times 2^f16_p lies in [2^-14, 2^13))
    bool f16 = false;
    int f16_p = 0;
    // the GEMM may plan its pre-pass forms (fp16, one-pass 8-bit); cleared to pin the
    // bf16 form
    bool prepass_forms = true;
    size_t rec_bytes() const { return (size_t)nb * gp * kRecBytes; }
};

inline Layout make_layout(int n, int k) {
    Layout l;
    l.n = n;
    l.k = k;
    l.kx = k;
    l.g = k / 64;
    l.nb = (n + 15) / 16;
    l.gp = (l.g + 1) / 2;
    return l;
}

// A gate|up pair of F rows each is tiled as one projection of pair_layout(F, K):
// block j holds gate rows 8j..8j+7 then up rows 8j..8j+7 (its N is 16 * ceil(F / 8)).
inline Layout pair_layout(int f, int k) { return make_layout(16 * ((f + 7) / 8), k); }

// MLX layout (device) -> tiled layout (device).  pair_rows = 0: one projection
// (w, s, b); pair_rows = F: the gate (w, s, b) and up (w_up, s_up, b_up) pair.
hipError_t launch_repack(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint32_t* w_up,
                         const uint16_t* s_up, const uint16_t* b_up, uint4* tiles, uint2* sb, const Layout& l,
                         int pair_rows, hipStream_t stream);

// Tiled layout -> fp32 W[N,K] row-major, w = fma(s, q, b); a pair gives [2, F, K].
hipError_t launch_dequantize(const uint4* tiles, const uint2* sb, float* out, const Layout& l, int pair_rows,
                             hipStream_t stream);

// 8-bit affine weights as two 4-bit planes over K' = 2K (q4_layout.hip): the layout l
// of such a handle is make_layout(N, 2K) (pair_layout(F, 2K) for a pair) with kx = K;
// its kernels read x [M, K] as x' = [x | x] (column c of x' is column c mod K of x).
hipError_t launch_repack8(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint32_t* w_up,
                          const uint16_t* s_up, const uint16_t* b_up, uint4* tiles, uint2* sb, const Layout& l,
                          int pair_rows, hipStream_t stream);
hipError_t launch_dequantize8(const uint4* tiles, const uint2* sb, float* out, const Layout& l, int pair_rows,
                              hipStream_t stream);
hipError_t launch_embed8(const uint4* tiles, const uint2* sb, const int32_t* ids, int count, void* out, bool out_f32,
                         const Layout& l, hipStream_t stream);

// out[t, :] = dequantized row ids[t] of a projection (fp32, or bf16 rounded once), t <
// count; ids outside [0, N) give zero rows.  out is 16-byte aligned, [count, K].
hipError_t launch_embed(const uint4* tiles, const uint2* sb, const int32_t* ids, int count, void* out, bool out_f32,
                        const Layout& l, hipStream_t stream);

// Output modes (q4_common.h OutMode): 0 bf16 y, 1 fp32 y, 2 bf16 GeGLU h, 3 fp32 GeGLU h,
// 4 / 5 the greedy lm_head (softcap, optional logits, per-block best keys).  n_out is
// F for the GeGLU modes (h is [M, F]) and unused otherwise.
struct OutParams;

// Decode path, any M in one launch (16-row slabs along the grid's y dimension).
hipError_t launch_decode(const uint4* tiles, const uint2* sb, const uint16_t* x, const OutParams& op, int m,
                         const Layout& l, hipStream_t stream);

// Decode kernel family (a process-wide choice for tests and benchmarks): 0 automatic,
// 1 the int8-limb kernels wherever they apply (1-8 rows of x), 2 the bf16 kernels only.
// set_decode_variant returns the previous choice (an atomic exchange).
int set_decode_variant(int v);
int decode_variant();

// One row of x on the int8 matrix cores (q4_limbs.hip): x split exactly into three
// int8 limbs per group once per workgroup, every output mode.  limb_lds_bytes is its
// dynamic LDS; the launch fails (hipErrorInvalidValue) when that exceeds the CU's LDS.
size_t limb_lds_bytes(const Layout& l);
hipError_t launch_decode_limbs(const uint4* tiles, const uint16_t* x, const OutParams& op, const Layout& l,
                               hipStream_t stream);
// 2-8 rows of x on the int8 matrix cores (rows padded to 2, 4 or 8); the launch fails
// (hipErrorInvalidValue) where limb_rows_lds_bytes exceeds the CU's LDS.
size_t limb_rows_lds_bytes(const Layout& l, int m);
// whether the automatic choice takes them for m rows of this layout (measured per shape)
bool limb_rows_preferred(const Layout& l, int m);
hipError_t launch_decode_limb_rows(const uint4* tiles, const uint16_t* x, const OutParams& op, int m,
                                   const Layout& l, hipStream_t stream);

// token[m] (and value[m] when not null) = argmax over the keys part[m][0..nb) left by
// the greedy modes, for m < rows.
hipError_t launch_greedy_reduce(const unsigned long long* part, int nb, int rows, int32_t* token, float* value,
                                hipStream_t stream);

// The fp16 form's pre-pass keeps a row's group sums in LDS: rows of x of at most this
// many groups.
constexpr int kPrepMaxGroups = 8192;
// Scale range of a built handle (the GEMM's fp16 form): out[0] the largest and out[1]
// the smallest biased exponent of its nonzero scales (a subnormal scale counts as 0;
// out[0] stays -1 when every scale is zero), out[2] the count of inf or NaN scales.
// `out` is device memory the caller sets to {-1, 255, 0} first.
hipError_t launch_scale_range(const uint2* sb, const Layout& l, int* out, hipStream_t stream);
// Sets l.f16 and l.f16_p from those three numbers.
void set_f16_form(Layout& l, const int range[3]);

// Prefill path: fp32-exact factored GEMM on the matrix cores.  `workspace` holds,
// for the 256-row tile and the pre-pass forms (fp16 on 256-row tiles, one-pass 8-bit
// on 128- and 256-row tiles), the group sums of x (and in the pre-pass forms x as
// fp16 and each row's power of two) and, when K is split over workgroups, the fp32
// partial sums (device memory, 256-byte aligned); an unsplit bf16-form plan of 64- or
// 128-row tiles needs none.  The plan is the cheapest whose workspace fits in
// `workspace_bytes`; gemm_workspace_bytes(m, l) is what the unconstrained plan
// needs, and with that much the launch runs the unconstrained plan.
struct GemmPlan {
    int bm = 256;            // output tile rows: 256, 128 or 64
    int bn = 256;            // output tile columns
    int splits = 1;          // workgroups along K per output tile
    int g_split = 0;         // groups per split (whole octets)
    size_t xaug_bytes = 0;   // group sums of x (256-row tiles)
    size_t part_bytes = 0;   // splits x M x N fp32 partial sums (0 when unsplit)
    bool f16 = false;        // fp16 form (256-row tiles of a handle whose scales allow it)
    bool q8 = false;         // one-pass 8-bit (128-row tiles of a two-plane handle)
    size_t x16_bytes = 0;    // fp16 and one-pass 8-bit forms: x scaled per row, as fp16 [M, kx]
    size_t rowexp_bytes = 0; // their rows' powers of two
    size_t total() const { return xaug_bytes + x16_bytes + rowexp_bytes + part_bytes; }
};
constexpr int kMaxSplits = 16;
constexpr size_t kMaxPartialBytes = (size_t)1 << 30;
GemmPlan plan_gemm(int m, const Layout& l, size_t max_workspace = ~(size_t)0);
size_t gemm_workspace_bytes(int m, const Layout& l);

// Compute units of the current device (cached per device).
int device_cus();
// gelu_table: kGeluTable bf16 values (q4_common.h) from launch_gelu_table, staged in
// LDS by the bf16 GeGLU epilogue (out_mode 2); may be null for the other modes.
hipError_t launch_gemm(const uint4* tiles, const uint2* sb, const uint16_t* x, void* y, int m, int out_mode,
                       int n_out, const Layout& l, void* workspace, size_t workspace_bytes,
                       const uint16_t* gelu_table, hipStream_t stream, const LoraEpilogue* lora = nullptr);
// Whether launch_gemm can add a LoRA delta of this rank in its epilogue for m rows
// within `workspace_bytes` (an unsplit plan; rank a multiple of 4 up to 32).
bool gemm_lora_epilogue(int m, const Layout& l, int rank, size_t workspace_bytes);

// Fills table[kGeluTable] with gelu of the bf16 patterns that need a table, in the
// bf16 op sequence.
hipError_t launch_gelu_table(uint16_t* table, hipStream_t stream);

// LoRA delta added in place to a projection output y [m, n] (bf16 or fp32) already
// holding the base product: part is fp32 scratch of lora_slices(k, m) x m x rank floats
// (x . A^T summed over slices of K), a [rank, k] and b [n, rank] fp32 on the device
// (q4_lora.hip).
constexpr int kLoraSlices = 8;
int lora_slices(int k, int m);
// Small M and rank: one fused launch that needs no part scratch (part may be null).
bool lora_fused(int m, int rank);
// a_hi, a_lo: A as bf16 high and low parts [ceil(rank / 16) * 16][k] (rows past rank
// zero), for the matrix-core x . A^T.
hipError_t launch_lora(const uint16_t* x, const float* a, const uint16_t* a_hi, const uint16_t* a_lo, const float* b,
                       float* part, void* y, int m, int n, int k, int rank, float scale, bool out_f32,
                       hipStream_t stream);
// Only the first step, part[slice][m][r] = x . A^T over lora_slices(k, m) slices of K
// (for a GEMM whose epilogue adds the delta).
hipError_t launch_lora_down(const uint16_t* x, const uint16_t* a_hi, const uint16_t* a_lo, float* part, int m,
                            int k, int rank, hipStream_t stream);

// Forward path choice (automatic mode): the decode kernels below kGemmMinRows rows,
// and beyond that while 16-row slabs x N x K stays at most kDecodeMaxSlabWork (K' = 2K
// for two-plane 8-bit handles).  The decode kernels' cost grows by one pass over the
// weights per 16-row slab (~0.24 us per million weights); the GEMM's starts at ~14 us
// (launch, tile prologue and epilogue, split-K reduction) and grows slowly at these
// sizes.  Measured as whole forwards (graph replays, each path pinned) on nine shapes
// (q, k, o, the fused qkv, gate, down, the gate|up pair, the full-attention o and k)
// at 32-256 rows: with any bound from 5e7 to 6e7 the choice is within 3% of the faster
// path everywhere (q 4096x3840: decode to 48 rows, 15.3 vs 16.3 us; GEMM from 56,
// 16.9 vs 18.3; the fused qkv 8192x3840 at 32 rows on the GEMM, 13.8 vs 19.9).
constexpr int kGemmMinRows = 32;
constexpr double kDecodeMaxSlabWork = 5.5e7;
// The slab bound was fitted on the Gemma shapes at 32-256 rows (the full-attention k,
// 512 x 3840, stays on decode to 448 rows); beyond 64 slabs the GEMM takes any shape.
constexpr long kDecodeMaxRows = 1024;
inline bool use_decode(long rows, const Layout& l, int gemm_min_rows) {
    if (gemm_min_rows > 0) return rows < gemm_min_rows;
    return rows < kGemmMinRows ||
           (rows <= kDecodeMaxRows && (double)((rows + 15) / 16) * (double)l.n * (double)l.k <= kDecodeMaxSlabWork);
}

}  // namespace q4
