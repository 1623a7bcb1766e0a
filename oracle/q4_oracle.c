/*
 * CPU oracle for MLX-format affine quantized matmul — TEST INFRASTRUCTURE ONLY.
 * See q4_oracle.h for the reference anchors and for what pins each function.
 */
#include "q4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f32_bits(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float v;
    memcpy(&v, &u, 4);
    return v;
}

uint16_t oracle_f32_to_bf16(float v) {
    uint32_t u = f32_bits(v);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0) {
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb; /* round to nearest, ties to even */
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t v) { return bits_f32((uint32_t)v << 16); }

static int valid_bits(int bits) { return bits == 2 || bits == 4 || bits == 8; }

static int valid_shape(int64_t n, int64_t k, int group, int bits) {
    if (n < 0 || k <= 0 || group <= 0 || !valid_bits(bits)) return 0;
    if (k % group != 0) return 0;
    if ((k * bits) % 32 != 0) return 0;
    if ((group * bits) % 32 != 0) return 0;
    return 1;
}

/*
 * MLX affine quantize, restated per group (MLX 0.31.2 CPU quantize loop; the
 * call site is the mlx-community artifact conversion that produced the
 * reference's weights, consumed at native_model.cc:349-362):
 *   scale = max((max-min)/n_bins, 1e-7); the sign makes the edge element the
 *   larger-magnitude end (edge = min -> positive scale, edge = max -> negative);
 *   q0 = rint(edge/scale); if q0 != 0 the scale is refined to edge/q0 and the
 *   bias is the edge, else bias = 0; q = clip(rint((w-bias)/scale), 0, n_bins)
 *   using the unrounded fp32 scale/bias; scale and bias are then stored as bf16.
 */
int oracle_affine_quantize(const float* w, int64_t n, int64_t k, int group, int bits,
                           uint32_t* wq, uint16_t* scales, uint16_t* biases) {
    if (!w || !wq || !scales || !biases || !valid_shape(n, k, group, bits)) return -1;
    const float n_bins = (float)((1 << bits) - 1);
    const float eps = 1e-7f;
    const int per_word = 32 / bits;
    const int64_t words_per_row = k / per_word;
    const int64_t groups_per_row = k / group;
    memset(wq, 0, (size_t)(n * words_per_row) * sizeof(uint32_t));
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t g = 0; g < groups_per_row; ++g) {
            const float* src = w + r * k + g * group;
            float w_min = INFINITY;
            float w_max = -INFINITY;
            for (int j = 0; j < group; ++j) {
                w_max = fmaxf(w_max, src[j]);
                w_min = fminf(w_min, src[j]);
            }
            const int min_is_edge = fabsf(w_min) > fabsf(w_max);
            float scale = fmaxf((w_max - w_min) / n_bins, eps);
            scale = min_is_edge ? scale : -scale;
            const float edge = min_is_edge ? w_min : w_max;
            const float q0 = rintf(edge / scale);
            float bias = 0.0f;
            if (q0 != 0.0f) {
                scale = edge / q0;
                bias = edge;
            }
            for (int j = 0; j < group; ++j) {
                float q = rintf((src[j] - bias) / scale);
                q = fminf(fmaxf(q, 0.0f), n_bins);
                const int64_t col = g * group + j;
                wq[r * words_per_row + col / per_word] |= ((uint32_t)q) << (bits * (col % per_word));
            }
            scales[r * groups_per_row + g] = oracle_f32_to_bf16(scale);
            biases[r * groups_per_row + g] = oracle_f32_to_bf16(bias);
        }
    }
    return 0;
}

/* q[r,c]: element c of row r sits in word c/(32/bits), lowest bits first
 * (native_model.cc:281-287 derives K from this packing). */
static inline uint32_t q_at(const uint32_t* wq, int64_t words_per_row, int64_t r, int64_t c, int bits) {
    const int per_word = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    return (wq[r * words_per_row + c / per_word] >> (bits * (c % per_word))) & mask;
}

int oracle_affine_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                             int64_t n, int64_t k, int group, int bits, float* out) {
    if (!wq || !scales || !biases || !out || !valid_shape(n, k, group, bits)) return -1;
    const int64_t words_per_row = k * bits / 32;
    const int64_t groups_per_row = k / group;
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t c = 0; c < k; ++c) {
            const float s = oracle_bf16_to_f32(scales[r * groups_per_row + c / group]);
            const float b = oracle_bf16_to_f32(biases[r * groups_per_row + c / group]);
            const float q = (float)q_at(wq, words_per_row, r, c, bits);
            out[r * k + c] = fmaf(s, q, b); /* s*q is exact in fp32, so one rounding */
        }
    }
    return 0;
}

int oracle_qmm_f64(const uint16_t* x, int64_t m, int64_t k, const uint32_t* wq,
                   const uint16_t* scales, const uint16_t* biases, int64_t n, int group,
                   int bits, double* y) {
    if (!x || !wq || !scales || !biases || !y || m < 0 || !valid_shape(n, k, group, bits)) return -1;
    const int64_t words_per_row = k * bits / 32;
    const int64_t groups_per_row = k / group;
    double* xrow = (double*)malloc((size_t)(k * (m > 0 ? m : 1)) * sizeof(double));
    if (!xrow) return -1;
    for (int64_t i = 0; i < m * k; ++i) xrow[i] = (double)oracle_bf16_to_f32(x[i]);
    int failed = 0;
    /* Rows of W are independent and each output is summed in column order by one
     * thread, so the result does not depend on the thread count. */
#pragma omp parallel reduction(| : failed)
    {
        double* wrow = (double*)malloc((size_t)k * sizeof(double));
        if (!wrow) failed = 1;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; ++r) {
            if (!wrow) continue;
            for (int64_t c = 0; c < k; ++c) {
                const double s = (double)oracle_bf16_to_f32(scales[r * groups_per_row + c / group]);
                const double b = (double)oracle_bf16_to_f32(biases[r * groups_per_row + c / group]);
                wrow[c] = s * (double)q_at(wq, words_per_row, r, c, bits) + b;
            }
            for (int64_t i = 0; i < m; ++i) {
                double acc = 0.0;
                const double* xi = xrow + i * k;
                for (int64_t c = 0; c < k; ++c) acc += xi[c] * wrow[c];
                y[i * n + r] = acc;
            }
        }
        free(wrow);
    }
    free(xrow);
    return failed ? -1 : 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

int oracle_qmm_f32(const uint16_t* x, int64_t m, int64_t k, const uint32_t* wq,
                   const uint16_t* scales, const uint16_t* biases, int64_t n, int group,
                   int bits, float* y, int threads) {
    if (!x || !wq || !scales || !biases || !y || m < 0 || !valid_shape(n, k, group, bits)) return -1;
    const int64_t words_per_row = k * bits / 32;
    const int64_t groups_per_row = k / group;
    float* xf = (float*)malloc((size_t)(k * (m > 0 ? m : 1)) * sizeof(float));
    if (!xf) return -1;
    for (int64_t i = 0; i < m * k; ++i) xf[i] = oracle_bf16_to_f32(x[i]);
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
    {
        float* wrow = (float*)malloc((size_t)k * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t r = 0; r < n; ++r) {
            if (!wrow) continue;
            const uint32_t* wr = wq + r * words_per_row;
            for (int64_t g = 0; g < groups_per_row; ++g) {
                const float s = oracle_bf16_to_f32(scales[r * groups_per_row + g]);
                const float b = oracle_bf16_to_f32(biases[r * groups_per_row + g]);
                const int per_word = 32 / bits;
                const uint32_t mask = (1u << bits) - 1u;
                for (int64_t c = g * group; c < (g + 1) * group; ++c) {
                    const uint32_t q = (wr[c / per_word] >> (bits * (c % per_word))) & mask;
                    wrow[c] = s * (float)q + b;
                }
            }
            for (int64_t i = 0; i < m; ++i) {
                const float* xi = xf + i * k;
                float acc = 0.0f;
#ifdef _OPENMP
#pragma omp simd reduction(+ : acc)
#endif
                for (int64_t c = 0; c < k; ++c) acc += xi[c] * wrow[c];
                y[i * n + r] = acc;
            }
        }
        free(wrow);
    }
    free(xf);
    (void)threads;
    return 0;
}
