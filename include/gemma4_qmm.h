/*
 * gemma4_qmm — MI355X (gfx950) affine 4-bit quantized linear layers behind a C ABI.
 *
 * Drop-in for the reference's quantized-linear call sites.  The reference issues
 * every projection as
 *     mlx::core::quantized_matmul(x, W, scales, biases, transpose=true,
 *                                 group_size, bits, "affine")
 * at native/gemma4_mlx/src/native_model.cc:349-362 (q/k/v/o and gate/up/down,
 * call sites :802,813,821,892,934,939,949 prefill, :993,1005,1009,1128,1318-1321
 * decode, :1158,1167,1171,1281,1366-1369 block/verify) and the lm_head at
 * native_model.cc:1782-1795.  Those weights are loaded once and stay resident
 * (native_model.cc:3550-3566), so the boundary here is a handle that owns the
 * device copy of one projection's weight triple, plus a forward call per step.
 *
 * Conventions follow the reference C ABI (native/gemma4_mlx/include/gemma4_mlx.h,
 * native/gemma4_mlx/src/runtime.cc):
 *   - every entry point returns a Gemma4Status (gemma4_mlx.h:12-21);
 *   - failures store a message in a thread-local buffer read back with
 *     gemma4_qmm_get_last_error (runtime.cc:46, :116-133, :816-823);
 *   - handles are opaque, carry a magic number checked on entry (runtime.cc:41-45),
 *     and have an explicit free (runtime.cc:900-912);
 *   - no C++ exception crosses the ABI (native_model.cc:3582-3588);
 *   - pointers are null-checked and sizes validated before use
 *     (spec/03-rust-mlx-ffi-contract.md "Safety checklist").
 *
 * Data formats (the MLX affine format, model_manifest.cc:101-162,
 * native_model.cc:281-287):
 *   weight  uint32 [N, K/8]  element k of a row is nibble k%8 of word k/8, lowest nibble first
 *   scales  bf16   [N, K/64] (raw bit patterns as uint16)
 *   biases  bf16   [N, K/64]
 *   w[n,k] = scales[n,k/64] * q[n,k] + biases[n,k/64]
 *   x       bf16   [M, K] row-major, device memory, 16-byte aligned
 *   y       bf16 or fp32 [M, N] row-major, device memory;  y = x . W^T
 * bits = 4 or 8 with group_size = 64 is accepted: the default of the reference's
 * Gemma 4 12B artifact and the only overrides its loader allows (model_manifest.cc:148).
 * With bits = 8 the weight is uint32 [N, K/4], code k in byte k%4 of word k/4, lowest
 * byte first; it is held as two 4-bit planes (q = 16*qh + ql) and runs on the same
 * kernels over 2K, which read x in place as [x | x].
 *
 * Streams are hipStream_t values passed as void* (NULL = the null stream).  All
 * device work is asynchronous on that stream.  A handle is immutable after
 * create, so forward/dequantize may run concurrently on several streams and
 * threads; create and free must not overlap use.  Scratch (split-K partial sums,
 * the 256-row GEMM tile's group sums, the greedy head's keys, LoRA's x.A^T) comes
 * from device memory the library keeps per (device, stream) and reuses call after
 * call in stream order.  A HIP graph that captured a call uses its capture stream's
 * memory, so replays of graphs captured on one stream must not overlap one another
 * or calls on that stream (replay them on one stream, or serialize).  When a call
 * needs more, the stream's memory grows; the outgrown buffer is freed unless a
 * capture used it.  The memory is held until gemma4_qmm_release_scratch or the end
 * of the process.
 */
#ifndef GEMMA4_QMM_H
#define GEMMA4_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEMMA4_QMM_ABI_VERSION 2u

/* Same codes as the reference status enum (gemma4_mlx.h:12-21); defined here only
 * when that header has not been included first. */
#ifndef GEMMA4_MLX_H
typedef enum Gemma4Status {
    GEMMA4_OK = 0,
    GEMMA4_ERR_INVALID_ARGUMENT = 1,
    GEMMA4_ERR_UNSUPPORTED_CONFIG = 2,
    GEMMA4_ERR_MODEL_LOAD = 3,
    GEMMA4_ERR_RUNTIME = 4,
    GEMMA4_ERR_MEMORY_GUARD = 5,
    GEMMA4_ERR_CACHE = 6,
    GEMMA4_ERR_ADAPTER = 7
} Gemma4Status;
#endif

typedef struct Gemma4QLinear Gemma4QLinear;

typedef enum Gemma4QmmDtype {
    GEMMA4_QMM_BF16 = 0,
    GEMMA4_QMM_F32 = 1
} Gemma4QmmDtype;

typedef struct Gemma4QmmVersionInfo {
    uint32_t abi_version;
    const char* backend_name;
    const char* backend_version;
} Gemma4QmmVersionInfo;

/* Shape and quantization of one projection (the reference's QuantizationSpec,
 * model_manifest.h:10-13, plus the weight's logical shape). */
typedef struct Gemma4QLinearDesc {
    uint32_t out_features; /* N */
    uint32_t in_features;  /* K, a multiple of group_size */
    uint32_t bits;         /* 4 or 8 */
    uint32_t group_size;   /* 64 */
} Gemma4QLinearDesc;

typedef struct Gemma4QLinearInfo {
    uint32_t out_features;
    uint32_t in_features;
    uint32_t bits;
    uint32_t group_size;
    uint64_t device_bytes; /* resident bytes of the tiled weight triple */
    int32_t device;        /* HIP device ordinal that holds it */
    uint32_t flags;        /* GEMMA4_QLINEAR_GEGLU_PAIR for a gate|up pair */
} Gemma4QLinearInfo;

#define GEMMA4_QLINEAR_GEGLU_PAIR 1u

/* Replaces gemma4_runtime_version (runtime.cc:805-814) for this library. */
Gemma4Status gemma4_qmm_runtime_version(Gemma4QmmVersionInfo* out);

/* Replaces gemma4_get_last_error (runtime.cc:816-823): copies this thread's last
 * error message (empty after a success) into buffer, NUL-terminated. */
Gemma4Status gemma4_qmm_get_last_error(char* buffer, size_t buffer_len);

/* Path choice of the forward calls in this process.  No counterpart in the
 * reference (MLX picks its own kernels); for tests and benchmarks that pin a path.
 *   0 (the default): automatic.  The decode kernels (16-row slabs, one pass over
 *     the weights per slab) below 32 rows, and beyond that while
 *     ceil(rows / 16) * N * K <= 5.5e7 (K' = 2K for 8-bit handles), the GEMM
 *     otherwise: for the Gemma 4 shapes the decode kernels are ahead of the GEMM's
 *     fixed costs up to 48 rows for 4096x3840, 112 for 2048x3840, 432 for 512x3840,
 *     and below 32 rows for 8192x3840 and the MLP projections.
 *   r > 0: the GEMM from r rows on, the decode kernels below.
 * Both paths meet the same accuracy contract; they sum in different orders, so the
 * last bits of some outputs differ between them.  Returns the previous setting.
 * Takes effect for calls issued after it returns (a process-wide atomic). */
uint32_t gemma4_qmm_set_gemm_min_rows(uint32_t rows);

/* Decode kernel family of the forward calls in this process.  No counterpart in the
 * reference; for tests and benchmarks that pin a kernel.
 *   0 (the default): automatic, chosen per shape.
 *   1: the int8 matrix-core kernels (x split exactly into three int8 limbs per
 *      64-column group) for every call of 1-8 rows they can run (x's limbs and the
 *      kernel's sums within a CU's LDS).
 *   2: the bf16 matrix-core kernels only.
 * All meet the same accuracy contract and sum in different orders.  Values above 2
 * are taken as 0.  Returns the previous setting; takes effect for calls issued after
 * it returns. */
uint32_t gemma4_qmm_set_decode_kernel(uint32_t variant);

/* GEMM (prefill) form of the forward calls in this process.  No counterpart in the
 * reference; for tests and benchmarks that compare the two.
 *   0 (the default): the plan may take the pre-pass forms, which scale x per row by
 *      a power of two into fp16: the fp16 form for 256-row tiles of handles whose
 *      scales allow it (every nonzero scale within 2^26 of the largest, none inf or
 *      NaN; weights expanded as s 2^p (q - 8), exact fp16 products with no per-group
 *      scale step), and for 8-bit handles the one-pass form (weights as 1024 + q from
 *      both planes, one pass over K instead of two 4-bit planes over 2K); the bf16
 *      form elsewhere.
 *   1: the bf16 form only (x as given, weights as 1 + q/16, scaled per group).
 * Both meet the same accuracy contract and sum in different orders.  Values above 1
 * are taken as 0.  Returns the previous setting; takes effect for calls issued after
 * it returns. */
uint32_t gemma4_qmm_set_gemm_form(uint32_t form);

/* Releases the device memory the library keeps for the scratch of calls on `stream`
 * on the current device (for hipStreamPerThread, the calling thread's), after waiting
 * for the stream's work.  No counterpart in the reference (MLX frees per call); for
 * long-running hosts that retire streams.  Graphs captured on that stream that used
 * the memory must not be replayed afterwards; later calls on the stream allocate
 * again.  A stream the library never used is a no-op. */
Gemma4Status gemma4_qmm_release_scratch(void* stream);

/* Load one projection's weight triple from HOST memory in MLX layout onto the
 * current HIP device (the per-prefix tensors the reference keeps in Impl::tensors,
 * native_model.cc:84-104, :3550-3566).  The host arrays may be freed on return. */
Gemma4Status gemma4_qlinear_create(const Gemma4QLinearDesc* desc, const uint32_t* weight,
                                   const uint16_t* scales, const uint16_t* biases,
                                   Gemma4QLinear** out);

/* Same, from DEVICE memory in MLX layout on the current device (weights already
 * uploaded by the caller).  The caller's buffers are read by a repack kernel on
 * `stream`; the call waits for that stream, so they may be freed on return and
 * the handle is usable on any stream. */
Gemma4Status gemma4_qlinear_create_device(const Gemma4QLinearDesc* desc, const uint32_t* weight_dev,
                                          const uint16_t* scales_dev, const uint16_t* biases_dev,
                                          void* stream, Gemma4QLinear** out);

/* Releases the device copy.  NULL is accepted (no-op), as for the reference frees. */
Gemma4Status gemma4_qlinear_free(Gemma4QLinear* linear);

Gemma4Status gemma4_qlinear_info(const Gemma4QLinear* linear, Gemma4QLinearInfo* out);

/* y[M,N] = x[M,K] . W^T — replaces quantized_linear (native_model.cc:349-362) and the
 * lm_head product (native_model.cc:1782-1795).  y_dtype BF16 is the model dtype;
 * F32 is the GEMMA4D_NATIVE_FORCE_FLOAT32 output (model_dtype, native_model.cc:330-340).
 * Accumulation is fp32.  rows == 0 is a no-op. */
Gemma4Status gemma4_qlinear_forward(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev,
                                    uint32_t rows, void* y_dev, Gemma4QmmDtype y_dtype);

/* Scratch bytes gemma4_qlinear_forward (or gemma4_qgeglu_forward, for a pair) takes
 * for `rows` rows under the current path choice: 0 on the decode path, else the GEMM
 * plan's group sums, its pre-pass forms' fp16 copy of x and row exponents, and its
 * split-K partial sums.  No counterpart in the reference.  When
 * it is at most 64 MiB, gemma4_qlinear_forward_noalloc runs the same plan, so the two
 * calls give identical bits. */
Gemma4Status gemma4_qlinear_scratch_bytes(const Gemma4QLinear* linear, uint32_t rows, uint64_t* out);

/* gemma4_qlinear_forward for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, hosts that forbid allocation): the same
 * arguments, results and kernels, with every scratch buffer taken from a static
 * 64 MiB device array that the library holds on each GPU it runs on until the
 * process ends.  No counterpart in the reference (its MLX ops allocate per call).
 * It calls no hipMalloc, hipFree or allocating library routine.  Scratch needs:
 * none on the decode path (gemma4_qmm_set_gemm_min_rows); on the GEMM path the table
 * of x's group sums that the 256-row tile and the pre-pass forms (fp16, one-pass
 * 8-bit) read (1 KiB per 16 rows, rounded up to the tile, and per 512 columns of K),
 * the pre-pass forms' fp16 copy of x (2 bytes per element) and row exponents (4 bytes
 * per row), and split-K partial
 * sums, only as far as the array has room (a cheaper tile, another form or fewer
 * splits than gemma4_qlinear_forward may choose, so the fp32 summation order, and with
 * it the last bits of some outputs, can differ from that call's; unsplit bf16-form
 * plans on the 64- and 128-row tiles need none), so no call is refused for want of
 * scratch.  Every call
 * on a GPU shares that GPU's array: calls that overlap in time on one GPU (other
 * streams, other threads) race and must be serialized by the caller. */
Gemma4Status gemma4_qlinear_forward_noalloc(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev,
                                            uint32_t rows, void* y_dev, Gemma4QmmDtype y_dtype);

/* The MLP block in one call — replaces the decode MLP's gate and up quantized_linear,
 * geglu and down quantized_linear (native_model.cc:1318-1321; prefill :934-949):
 *     h = geglu(x . Wg^T, x . Wu^T)   (bf16 [rows, F], written to h_dev)
 *     y = h . Wd^T                    (bf16 [rows, N_down])
 * gate_up is a pair from gemma4_qgeglu_create, down a projection whose in_features is
 * the pair's F, on the same device.  It queues the pair's launch and then down's (the
 * kernels of gemma4_qgeglu_forward and gemma4_qlinear_forward, so the same bits).
 * y_dtype must be BF16 (the bf16 model dtype; under the float32 override h is fp32,
 * which these kernels do not take as x): GEMMA4_ERR_UNSUPPORTED_CONFIG otherwise.
 * h_dev is 16-byte aligned. */
Gemma4Status gemma4_qmlp_forward(const Gemma4QLinear* gate_up, const Gemma4QLinear* down, void* stream,
                                 const uint16_t* x_dev, uint32_t rows, uint16_t* h_dev, void* y_dev,
                                 Gemma4QmmDtype y_dtype);

/* Writes the fp32 dequantized weight W[N,K] = s*q + b (row-major) to w_dev —
 * mlx::core::dequantize (native_model.cc:364-376) with a float32 result.  Bit-exact:
 * the product s*q is exact in fp32, so the value is unique.  For a gate|up pair the
 * output is [2, F, K]: the gate rows, then the up rows. */
Gemma4Status gemma4_qlinear_dequantize(const Gemma4QLinear* linear, void* stream, float* w_dev);

/* ---- LoRA adapters on a quantized projection ----
 * Replaces quantized_linear's add_lora_delta_if_active (native_model.cc:316-328):
 *     y = model_dtype(base + model_dtype((float32(x) . A^T) . B^T * scale))
 * with the adapter module's A [rank, K] (lora_A.weight) and B [N, rank]
 * (lora_B.weight) as float32 and scale = alpha / rank (native_model.cc:3376-3426).
 * With y_dtype BF16 the base output and the delta are each rounded to bf16 and added
 * in bf16 (the scale is bf16, model_scalar); F32 keeps everything fp32. */
typedef struct Gemma4QLora Gemma4QLora;

/* Copies A and B (host fp32, row-major) to the current device. */
Gemma4Status gemma4_qlora_create(const float* a, const float* b, uint32_t rank, uint32_t in_features,
                                 uint32_t out_features, float scale, Gemma4QLora** out);
Gemma4Status gemma4_qlora_free(Gemma4QLora* lora);

/* gemma4_qlinear_forward plus the adapter's delta; lora NULL is the plain forward.
 * The adapter must match the projection's K and N and live on its device.  Up to 4
 * rows with rank up to 64: one fused launch and no scratch; otherwise scratch of at
 * most 8 * rows * rank * 4 bytes (x . A^T summed over up to eight slices of K).  Where
 * the forward runs on an unsplit GEMM plan and the rank is a multiple of 4 up to 32,
 * x . A^T is formed first and the GEMM's epilogue adds the delta (t . B^T on the bf16
 * matrix cores from high and low bf16 parts of t and B, within about 2^-16 of the fp32
 * sum, then the same roundings); otherwise the delta is added after the forward. */
Gemma4Status gemma4_qlinear_forward_lora(const Gemma4QLinear* linear, const Gemma4QLora* lora, void* stream,
                                         const uint16_t* x_dev, uint32_t rows, void* y_dev, Gemma4QmmDtype y_dtype);

/* Quantized embedding gather — replaces quantized_embedding (native_model.cc:364-376:
 * take of the embed_tokens triple's rows, then dequantize; the same tied triple the
 * lm_head uses).  out[t, :] = s * q + b of row ids[t], for t < count:
 *   ids_dev int32 [count] on the device; ids outside [0, N) give rows of zeros
 *   out_dev [count, K] of dtype, 16-byte aligned: F32 is bit-exact (as
 *   gemma4_qlinear_dequantize); BF16 is that fp32 value rounded once (to nearest even). */
Gemma4Status gemma4_qlinear_embed(const Gemma4QLinear* linear, void* stream, const int32_t* ids_dev, uint32_t count,
                                  void* out_dev, Gemma4QmmDtype dtype);

/* Greedy lm_head: the product, the final-logit softcap and argmax in one call —
 * replaces target_logits_for_hidden (native_model.cc:1782-1795: quantized_matmul, then
 * tanh(logits / 30) * 30) followed by argmax over the vocabulary (native_model.cc:3734,
 * :3825, :3934; per row at :4114, :4242) and the max logit (greedy_logit_for_vector_logits).
 *   token_dev [rows] int32   index of the first maximum of row m's softcapped logits
 *   value_dev [rows] float   that maximum (optional, NULL to skip)
 *   logits_dev [rows, N]     the softcapped logits in dtype (optional, NULL to skip)
 * softcap 0 skips the softcap.  With dtype BF16 the logits and every softcap op are
 * rounded to bf16 as the reference's bf16 array ops are; F32 keeps fp32.  rows <= 16
 * (a decode step or a verify block, gemma4_mlx.h:77-79).  Deterministic: ties go to
 * the lowest index whatever the execution order.  Uses a stream-ordered scratch of
 * rows * ceil(N/16) * 8 bytes. */
Gemma4Status gemma4_qlinear_forward_greedy(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev,
                                           uint32_t rows, float softcap, void* logits_dev, Gemma4QmmDtype dtype,
                                           int32_t* token_dev, float* value_dev);

/* ---- Fused gate|up projection with the GeGLU epilogue ----
 * Replaces the reference's MLP front half, two quantized_linear calls on the same
 * input followed by geglu (native_model.cc:934-949 prefill, :1318-1321 decode, and
 * geglu itself at native_model.cc:378-386):
 *     h[M,F] = geglu(x . Wg^T, x . Wu^T),  geglu(g, u) = 0.5*g*(1+tanh(c1*(g+c2*g^3)))*u
 * in one pass over both weight matrices, without writing gate and up to memory.
 * With h_dtype BF16 the qmm outputs and every GeGLU op are rounded to bf16 as the
 * reference's bf16 array ops are (constants bf16(0.7978845608), bf16(0.044715));
 * with F32 everything stays fp32 (the GEMMA4D_NATIVE_FORCE_FLOAT32 path).  The pair
 * is one Gemma4QLinear handle (freed with gemma4_qlinear_free; info reports
 * out_features = F and flags = GEMMA4_QLINEAR_GEGLU_PAIR); desc describes one of
 * the two projections (out_features = F, the same K, bits and group size for both). */
Gemma4Status gemma4_qgeglu_create(const Gemma4QLinearDesc* desc, const uint32_t* gate_weight,
                                  const uint16_t* gate_scales, const uint16_t* gate_biases, const uint32_t* up_weight,
                                  const uint16_t* up_scales, const uint16_t* up_biases, Gemma4QLinear** out);

/* Same, from device memory in MLX layout (as gemma4_qlinear_create_device). */
Gemma4Status gemma4_qgeglu_create_device(const Gemma4QLinearDesc* desc, const uint32_t* gate_weight_dev,
                                         const uint16_t* gate_scales_dev, const uint16_t* gate_biases_dev,
                                         const uint32_t* up_weight_dev, const uint16_t* up_scales_dev,
                                         const uint16_t* up_biases_dev, void* stream, Gemma4QLinear** out);

/* h[M,F] = geglu(x . Wg^T, x . Wu^T) on a handle from gemma4_qgeglu_create*.  x as for
 * gemma4_qlinear_forward; h is [rows, F] of h_dtype in device memory.  A plain
 * projection handle is rejected here, and a pair is rejected by gemma4_qlinear_forward. */
Gemma4Status gemma4_qgeglu_forward(const Gemma4QLinear* pair, void* stream, const uint16_t* x_dev, uint32_t rows,
                                   void* h_dev, Gemma4QmmDtype h_dtype);

#ifdef __cplusplus
}
#endif

#endif /* GEMMA4_QMM_H */
