// MLX affine quantizer and dequantizer (load-time ops, not on the decode path).
//
// quantize: mx.quantize(w_f32, group_size=64, bits) as called at
// src/shardcompute/parallel/quantized_linear.py:116-120 / :353-357 and
// parallel/embedding.py:303-307.  Per group of 64 values, in fp32:
//     scale = max((wmax - wmin) / n_bins, 1e-7)
//     edge  = |wmin| > |wmax| ? wmin : wmax   (scale negated when edge = wmax)
//     q0    = rint(edge / scale);  if q0 != 0: scale = edge / q0, bias = edge
//                                  else:       bias = 0
//     q     = clamp(rint((w - bias) / scale), 0, n_bins)
// packed LSB-first into uint32 words; scale and bias are stored as bf16 (RNE).
// Division is IEEE (HIP's default correctly rounded fp32 divide), rint is
// round-half-even, so the codes equal a float32 numpy evaluation bit for bit.
//
// dequantize: mx.dequantize (parallel/embedding.py:369-379), bf16(fma(s, q, b)).
#include "sc_common.h"

namespace sc {

template <int BITS>
__global__ void __launch_bounds__(256) quantize_affine_kernel(const float *w, int64_t rows, int64_t K,
                                                              uint32_t *wq, uint16_t *s_out, uint16_t *b_out) {
    const int64_t G = K / 64;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * G) return;
    const int64_t r = idx / G, g = idx - (idx / G) * G;
    const float *src = w + r * K + g * 64;
    float wmax = src[0], wmin = src[0];
    for (int i = 1; i < 64; ++i) {
        wmax = fmaxf(wmax, src[i]);
        wmin = fminf(wmin, src[i]);
    }
    const float n_bins = (float)((1 << BITS) - 1);
    float scale = fmaxf((wmax - wmin) / n_bins, 1e-7f);
    const bool use_min = fabsf(wmin) > fabsf(wmax);
    scale = use_min ? scale : -scale;
    const float edge = use_min ? wmin : wmax;
    const float q0 = rintf(edge / scale);
    float bias = 0.f;
    if (q0 != 0.f) {
        scale = edge / q0;
        bias = edge;
    }
    constexpr int PF = 32 / BITS;
    uint32_t *dst = wq + r * (K / PF) + g * (64 / PF);
    for (int wi = 0; wi < 64 / PF; ++wi) {
        uint32_t word = 0;
        for (int j = 0; j < PF; ++j) {
            float q = rintf((src[wi * PF + j] - bias) / scale);
            q = fminf(fmaxf(q, 0.f), n_bins);
            word |= ((uint32_t)q) << (BITS * j);
        }
        dst[wi] = word;
    }
    s_out[idx] = (uint16_t)f2bf(scale);
    b_out[idx] = (uint16_t)f2bf(bias);
}

template <int BITS>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                                                         int64_t rows, int64_t K, uint16_t *out) {
    constexpr int PF = 32 / BITS;
    const int64_t words = rows * (K / PF);
    const int64_t G = K / 64;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / (K / PF);
        const int64_t k0 = (i - r * (K / PF)) * PF;
        const float sf = bf2f(s[r * G + k0 / 64]);
        const float bf = bf2f(b[r * G + k0 / 64]);
        const uint32_t w = wq[i];
        uint16_t *dst = out + r * K + k0;
        for (int j = 0; j < PF; ++j)
            dst[j] = (uint16_t)f2bf(fmaf(sf, (float)((w >> (BITS * j)) & ((1u << BITS) - 1u)), bf));
    }
}

int launch_quantize(const float *w, int64_t rows, int64_t K, int bits, uint32_t *wq, uint16_t *s, uint16_t *b,
                    hipStream_t stream) {
    const int64_t n = rows * (K / 64);
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    if (bits == 4)
        hipLaunchKernelGGL(quantize_affine_kernel<4>, grid, block, 0, stream, w, rows, K, wq, s, b);
    else
        hipLaunchKernelGGL(quantize_affine_kernel<8>, grid, block, 0, stream, w, rows, K, wq, s, b);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_dequantize(const uint32_t *wq, const uint16_t *s, const uint16_t *b, int64_t rows, int64_t K, int bits,
                      uint16_t *out, hipStream_t stream) {
    const int64_t words = rows * K * bits / 32;
    int64_t blocks = (words + 255) / 256;
    const int64_t cap = (int64_t)device_info().num_cus * 32;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    if (bits == 4)
        hipLaunchKernelGGL(dequantize_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, wq, s, b, rows, K, out);
    else
        hipLaunchKernelGGL(dequantize_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, stream, wq, s, b, rows, K, out);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // namespace sc
