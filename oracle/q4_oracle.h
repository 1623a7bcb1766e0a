/*
 * CPU oracle for MLX-format affine quantized matmul — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the arithmetic that the reference reaches
 * through mlx::core::quantize / dequantize / quantized_matmul(mode="affine").
 * Only tests, the smoke check and the benchmark's CPU-baseline leg may link it;
 * the product library never does.
 *
 * Reference anchors (paths relative to the reference checkout):
 *   native/gemma4_mlx/src/native_model.cc:349-362   quantized_linear -> quantized_matmul(transpose=true, g, bits, "affine")
 *   native/gemma4_mlx/src/native_model.cc:364-376   quantized_embedding -> dequantize
 *   native/gemma4_mlx/src/native_model.cc:281-287   K = packed_cols * 32 / bits
 *   native/gemma4_mlx/src/native_model.cc:1782-1795 lm_head through the same op
 *   native/gemma4_mlx/src/model_manifest.cc:148     group 64, bits 4 or 8
 *   scripts/xr54_dequant_assistant.py:103-126       dequantize(..., dtype=float32) with float32 scales/biases
 * The arithmetic itself lives in MLX 0.31.2 (not vendored); the restated
 * algorithm follows MLX's published CPU quantize loop (see q4_oracle.c).
 *
 * Parity pins (tests/test_oracle.py, tests/test_golden.py):
 *   pack layout        : pack/unpack identity, brute-force bit positions, hand vectors
 *   dequantize (fp32)  : closed form s*q+b is exact in fp32 -> exhaustive over q, sampled s/b
 *   qmm (fp64 accum)   : brute-force loops, numpy/torch float64 matmul of the dequantized W,
 *                        zero/constant-group closed forms
 *   quantize           : invariants (q range, edge element reconstruction, error <= |s|/2),
 *                        hand-derived known-answer groups
 * Parity unpinned (needs an MLX import, absent here): the exact bf16 bits MLX's own
 * quantize writes for s/b, MLX's CPU accumulation order, bf16-output dequantize.
 */
#ifndef HELIOS_Q4_ORACLE_H
#define HELIOS_Q4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> f32 with round-to-nearest-even (NaN stays NaN). */
uint16_t oracle_f32_to_bf16(float v);
float oracle_bf16_to_f32(uint16_t v);

/* Affine quantize W[N,K] (fp32 values) with group size g and bits in {2,4,8}.
 * Writes packed uint32 [N, K*bits/32], scales/biases bf16 [N, K/g].
 * Returns 0 on success, -1 on bad arguments. */
int oracle_affine_quantize(const float* w, int64_t n, int64_t k, int group, int bits,
                           uint32_t* wq, uint16_t* scales, uint16_t* biases);

/* Dequantize to fp32: out[n,k] = s*q + b evaluated in fp32 (exact product). */
int oracle_affine_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                             int64_t n, int64_t k, int group, int bits, float* out);

/* y[m,n] = sum_k x[m,k] * (s*q+b), x bf16 [M,K], accumulation in double,
 * result left in double (caller rounds once). */
int oracle_qmm_f64(const uint16_t* x, int64_t m, int64_t k, const uint32_t* wq,
                   const uint16_t* scales, const uint16_t* biases, int64_t n, int group,
                   int bits, double* y);

/* The CPU baseline loop: per output row, per group, dequantize in fp32 and dot in
 * fp32, parallel over N with OpenMP when compiled with -fopenmp. Output fp32. */
int oracle_qmm_f32(const uint16_t* x, int64_t m, int64_t k, const uint32_t* wq,
                   const uint16_t* scales, const uint16_t* biases, int64_t n, int group,
                   int bits, float* y, int threads);

/* Number of OpenMP threads the library would use (1 when built without OpenMP). */
int oracle_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif
