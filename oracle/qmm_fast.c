/*
 * A vectorised C/OpenMP CPU restatement of the quantized matmul — TEST
 * INFRASTRUCTURE ONLY: the timed CPU baseline beside the GPU measurements (the
 * reference runs mx.quantized_matmul on MLX's CPU backend, which is not available
 * here; this is not MLX).  Checked against the fp64 oracle (oref_qmm_bf16) by the
 * CPU tests.
 *
 * Same contraction as oref_qmm_bf16 (src/shardcompute/parallel/quantized_linear.py:
 * 168-180), arranged the way a CPU implementation would run it: fp32 accumulation,
 *     y[m,n] = sum_g ( s[n,g] * sum_{k in g} x[m,k] q[n,k] + b[n,g] * sum_{k in g} x[m,k] )
 * with x converted to fp32 once and its group sums precomputed, each weight row's
 * group of codes unpacked to fp32 once and reused for every row of x, and the
 * 64-element dot products written so the compiler vectorises them (AVX2 + FMA).
 * Threads split the weight rows.  Output bf16 (round to nearest even), the
 * optional bias added to the rounded product and rounded again.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float f_of_bf16(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t bf16_of_f(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

int oref_qmm_fast_bf16(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                       const uint16_t *bias, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                       int group_size, int threads) {
    if (bits != 4 && bits != 8) return -1;
    if (group_size != 64 || K % 64) return -2;
    const int pf = 32 / bits;
    const int64_t G = K / 64, W = K / pf;
    float *xf = (float *)malloc(sizeof(float) * (size_t)(M * K));
    float *xs = (float *)malloc(sizeof(float) * (size_t)(M * G));
    if (!xf || !xs) {
        free(xf);
        free(xs);
        return -3;
    }
    for (int64_t i = 0; i < M * K; ++i) xf[i] = f_of_bf16(x[i]);
    for (int64_t m = 0; m < M; ++m)
        for (int64_t g = 0; g < G; ++g) {
            float t = 0.f;
            for (int k = 0; k < 64; ++k) t += xf[m * K + g * 64 + k];
            xs[m * G + g] = t;
        }
    int err = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)M);
        if (!acc) {
#pragma omp atomic write
            err = -3;
        } else {
#pragma omp for schedule(static)
            for (int64_t n = 0; n < N; ++n) {
                const uint32_t *wr = wq + n * W;
                for (int64_t m = 0; m < M; ++m) acc[m] = 0.f;
                for (int64_t g = 0; g < G; ++g) {
                    float q[64];
                    const uint32_t *wg = wr + g * (64 / pf);
                    if (bits == 4) {
                        for (int k = 0; k < 64; ++k) q[k] = (float)((wg[k >> 3] >> (4 * (k & 7))) & 15u);
                    } else {
                        for (int k = 0; k < 64; ++k) q[k] = (float)((wg[k >> 2] >> (8 * (k & 3))) & 255u);
                    }
                    const float s = f_of_bf16(scales[n * G + g]), b = f_of_bf16(biases[n * G + g]);
                    for (int64_t m = 0; m < M; ++m) {
                        const float *xr = xf + m * K + g * 64;
                        float d = 0.f;
#pragma omp simd reduction(+ : d)
                        for (int k = 0; k < 64; ++k) d += xr[k] * q[k];
                        acc[m] += s * d + b * xs[m * G + g];
                    }
                }
                for (int64_t m = 0; m < M; ++m) {
                    uint16_t o = bf16_of_f(acc[m]);
                    if (bias) o = bf16_of_f(f_of_bf16(o) + f_of_bf16(bias[n]));
                    y[m * N + n] = o;
                }
            }
            free(acc);
        }
    }
    free(xf);
    free(xs);
    return err;
}
