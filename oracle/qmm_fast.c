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
 * 64-element dot products as 8-wide FMA chains (AVX2 + FMA intrinsics: the codes are
 * unpacked with variable shifts, eight per instruction).
 * Threads split the weight rows.  Output bf16 (round to nearest even), the
 * optional bias added to the rounded product and rounded again.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#endif

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
        float *acc = (float *)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1));
        int ok = acc != NULL;
        if (!ok) {
#pragma omp atomic write
            err = -3;
        }
        {
            // every thread takes part in the loop (a worksharing construct); one
            // without its buffers skips its rows and the call returns -3
#pragma omp for schedule(static)
            for (int64_t n = 0; n < N; ++n) {
                if (!ok) continue;
                const uint32_t *wr = wq + n * W;
                for (int64_t m = 0; m < M; ++m) acc[m] = 0.f;
                for (int64_t g = 0; g < G; ++g) {
                    const uint32_t *wg = wr + g * (64 / pf);
                    const float s = f_of_bf16(scales[n * G + g]), b = f_of_bf16(biases[n * G + g]);
#if defined(__AVX2__) && defined(__FMA__)
                    // the group's 64 codes as 8 vectors of 8 floats (k order), then one
                    // 8-wide FMA chain per row of x
                    __m256 q[8];
                    if (bits == 4) {
                        const __m256i sh = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
                        for (int j = 0; j < 8; ++j)
                            q[j] = _mm256_cvtepi32_ps(_mm256_and_si256(
                                _mm256_srlv_epi32(_mm256_set1_epi32((int)wg[j]), sh), _mm256_set1_epi32(15)));
                    } else {
                        const __m256i sh = _mm256_setr_epi32(0, 8, 16, 24, 0, 8, 16, 24);
                        for (int j = 0; j < 8; ++j) {
                            const __m256i v = _mm256_setr_epi32((int)wg[2 * j], (int)wg[2 * j], (int)wg[2 * j],
                                                                (int)wg[2 * j], (int)wg[2 * j + 1], (int)wg[2 * j + 1],
                                                                (int)wg[2 * j + 1], (int)wg[2 * j + 1]);
                            q[j] = _mm256_cvtepi32_ps(_mm256_and_si256(_mm256_srlv_epi32(v, sh), _mm256_set1_epi32(255)));
                        }
                    }
                    for (int64_t m = 0; m < M; ++m) {
                        const float *xr = xf + m * K + g * 64;
                        __m256 d8 = _mm256_mul_ps(_mm256_loadu_ps(xr), q[0]);
                        for (int j = 1; j < 8; ++j) d8 = _mm256_fmadd_ps(_mm256_loadu_ps(xr + 8 * j), q[j], d8);
                        const __m128 h = _mm_add_ps(_mm256_castps256_ps128(d8), _mm256_extractf128_ps(d8, 1));
                        const __m128 h2 = _mm_add_ps(h, _mm_movehl_ps(h, h));
                        const float d = _mm_cvtss_f32(_mm_add_ss(h2, _mm_shuffle_ps(h2, h2, 1)));
                        acc[m] += s * d + b * xs[m * G + g];
                    }
#else
                    float q[64];
                    if (bits == 4) {
                        for (int k = 0; k < 64; ++k) q[k] = (float)((wg[k >> 3] >> (4 * (k & 7))) & 15u);
                    } else {
                        for (int k = 0; k < 64; ++k) q[k] = (float)((wg[k >> 2] >> (8 * (k & 3))) & 255u);
                    }
                    for (int64_t m = 0; m < M; ++m) {
                        const float *xr = xf + m * K + g * 64;
                        float d = 0.f;
#pragma omp simd reduction(+ : d)
                        for (int k = 0; k < 64; ++k) d += xr[k] * q[k];
                        acc[m] += s * d + b * xs[m * G + g];
                    }
#endif
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
