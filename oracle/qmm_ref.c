/*
 * C/OpenMP restatement of the reference's quantized matmul and masked gather —
 * TEST INFRASTRUCTURE ONLY (the oracle and the timed CPU baseline).
 *
 * oref_qmm_bf16 restates mx.quantized_matmul(x, wq, s, b, transpose=True,
 * group_size, bits) as called at src/shardcompute/parallel/quantized_linear.py:168-176
 * followed by the optional "+ self.bias" of :179-180:
 *     y[m,n] = bf16( sum_k x[m,k] * (s[n,k/gs] * q[n,k] + b[n,k/gs]) )
 *     y[m,n] = bf16( y[m,n] + bias[n] )            (when bias != NULL)
 * q[n,k] is element k % (32/bits) of word wq[n, k / (32/bits)], least
 * significant bits first.  Accumulation is in double, per output.
 *
 * oref_vocab_gather_bf16 restates src/shardcompute/parallel/embedding.py:322-356
 * on a bf16 table: rows of in-shard ids are copied bit for bit, other rows are +0.
 *
 * Built by oracle/Makefile with gcc; bound from oracle/cref.py.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

int oref_qmm_bf16(const uint16_t *x, const uint32_t *wq, const uint16_t *scales,
                  const uint16_t *biases, const uint16_t *bias, uint16_t *y,
                  int64_t M, int64_t N, int64_t K, int bits, int group_size, int threads) {
    if (bits != 4 && bits != 8) return -1;
    const int pf = 32 / bits;
    if (K % group_size || group_size % pf) return -2;
    const int64_t G = K / group_size;
    const int64_t W = K / pf;
    const uint32_t mask = (1u << bits) - 1u;
    (void)threads;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            const uint32_t *wr = wq + n * W;
            const uint16_t *sr = scales + n * G;
            const uint16_t *br = biases + n * G;
            for (int64_t m = 0; m < M; ++m) {
                const uint16_t *xr = x + m * K;
                double acc = 0.0;
                for (int64_t g = 0; g < G; ++g) {
                    const double s = bf16_to_f32(sr[g]);
                    const double b = bf16_to_f32(br[g]);
                    const int64_t w0 = g * group_size / pf;
                    for (int64_t w = w0; w < w0 + group_size / pf; ++w) {
                        uint32_t word = wr[w];
                        for (int j = 0; j < pf; ++j) {
                            const uint32_t q = word & mask;
                            word >>= bits;
                            acc += (double)bf16_to_f32(xr[w * pf + j]) * (s * (double)q + b);
                        }
                    }
                }
                uint16_t out = f32_to_bf16((float)acc);
                if (bias) out = f32_to_bf16(bf16_to_f32(out) + bf16_to_f32(bias[n]));
                y[m * N + n] = out;
            }
        }
    }
    return 0;
}

int oref_vocab_gather_bf16(const void *ids, int ids_is_int64, int64_t T, const uint16_t *table,
                           int64_t v_local, int64_t D, int64_t vocab_start, uint16_t *out,
                           int threads) {
    if (v_local <= 0 || D <= 0) return -1;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int64_t t = 0; t < T; ++t) {
        const int64_t id = ids_is_int64 ? ((const int64_t *)ids)[t] : (int64_t)((const int32_t *)ids)[t];
        uint16_t *dst = out + t * D;
        if (id >= vocab_start && id < vocab_start + v_local) {
            memcpy(dst, table + (id - vocab_start) * D, (size_t)D * 2);
        } else {
            memset(dst, 0, (size_t)D * 2);
        }
    }
    return 0;
}
