// Kernel B: LDS-staged dequant -> bf16 MFMA GEMM for prefill-sized batches.
//
// Same contraction as kernel A (mx.quantized_matmul(..., transpose=True),
// src/shardcompute/parallel/quantized_linear.py:168-176), for M >= 64 rows of x:
//     y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
//
// Workgroup tile BM x BN, stepping K one quantization group (64) at a time.
// Per step every thread issues its global loads for the next group (x tile
// rows, packed weight bytes, one scale/bias pair) before the MFMAs of the
// current group run; the weights are dequantized in registers to
// bf16(s * q + b) and written, with the x tile, into the other half of a
// double-buffered LDS area.  Waves (2 x 2) each own a (BM/2) x (BN/2) sub-tile
// computed with v_mfma_f32_32x32x16_bf16, fp32 accumulation; the epilogue rounds
// to bf16 and adds the optional linear bias after that rounding (the reference
// adds the bias to the bf16 matmul result, quantized_linear.py:179-180).
#include "sc_common.h"

namespace sc {

struct GemmArgs {
    const uint16_t *x;
    const uint32_t *wq;
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    int M, N, K, G;
};

namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;                 // one quantization group
constexpr int ROW_U4 = BK * 2 / 16 + 1;  // 8 uint4 of bf16 per row + 1 pad
constexpr int TILE_U4 = BM * ROW_U4;     // A tile (BM rows) == B tile (BN rows)
constexpr int THREADS = 256;

template <int BITS>
struct WLoad {
    uint4 v[BITS / 4];   // codes for 32 k of one row (W4: 16 B, W8: 32 B)
};

}  // namespace

template <int BITS>
__global__ void __launch_bounds__(THREADS) qgemm_mfma_kernel(GemmArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint4 *As = reinterpret_cast<uint4 *>(smem);   // [2][BM][ROW_U4]
    uint4 *Bs = As + 2 * TILE_U4;                  // [2][BN][ROW_U4]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int M = a.M, N = a.N, K = a.K, G = a.G;

    // x tile: 128 rows x 8 uint4 = 1024 uint4, 4 per thread
    const uint16_t *xrow[4];
    int xr[4], xc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + THREADS * i;
        xr[i] = idx >> 3;
        xc[i] = idx & 7;
        xrow[i] = a.x + (size_t)min(m0 + xr[i], M - 1) * K + xc[i] * 8;
    }
    // weights: thread -> (row, half): 32 k of one row per group
    const int wr = tid >> 1;
    const int wh = tid & 1;
    const int wn_row = min(n0 + wr, N - 1);
    const uint4 *wbase = reinterpret_cast<const uint4 *>(a.wq) + (size_t)wn_row * ((size_t)K * BITS / 128);
    const uint16_t *srow = a.s + (size_t)wn_row * G;
    const uint16_t *brow = a.b + (size_t)wn_row * G;

    uint4 xv[4];
    WLoad<BITS> wv;
    uint32_t sv, bv;
    auto gload = [&](int g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const uint4 *>(xrow[i] + (size_t)g * BK);
#pragma unroll
        for (int p = 0; p < BITS / 4; ++p) wv.v[p] = wbase[(size_t)g * (BITS / 2) + wh * (BITS / 4) + p];
        sv = srow[g];
        bv = brow[g];
    };
    auto lstore = [&](int buf) {
        uint4 *A = As + buf * TILE_U4;
        uint4 *B = Bs + buf * TILE_U4;
#pragma unroll
        for (int i = 0; i < 4; ++i) A[xr[i] * ROW_U4 + xc[i]] = xv[i];
        const float sf = bf2f(sv), bf = bf2f(bv);
        uint32_t out[16];
        if (BITS == 4) {
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                const uint32_t w = wi == 0 ? wv.v[0].x : wi == 1 ? wv.v[0].y : wi == 2 ? wv.v[0].z : wv.v[0].w;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float q0 = (float)((w >> (8 * j)) & 0xFu);
                    const float q1 = (float)((w >> (8 * j + 4)) & 0xFu);
                    out[wi * 4 + j] = pack_bf16x2(fmaf(sf, q0, bf), fmaf(sf, q1, bf));
                }
            }
        } else {
#pragma unroll
            for (int wi = 0; wi < 8; ++wi) {
                const uint4 u = wv.v[wi >> 2];
                const uint32_t w = (wi & 3) == 0 ? u.x : (wi & 3) == 1 ? u.y : (wi & 3) == 2 ? u.z : u.w;
                out[wi * 2 + 0] = pack_bf16x2(fmaf(sf, ubyte_f32(w, 0), bf),
                                              fmaf(sf, ubyte_f32(w, 1), bf));
                out[wi * 2 + 1] = pack_bf16x2(fmaf(sf, ubyte_f32(w, 2), bf),
                                              fmaf(sf, ubyte_f32(w, 3), bf));
            }
        }
        uint4 *dst = B + wr * ROW_U4 + wh * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = make_uint4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16_t{};

    const int li = lane & 31;
    const int lh = lane >> 5;

    gload(0);
    lstore(0);
    __syncthreads();
    for (int g = 0; g < G; ++g) {
        const int buf = g & 1;
        if (g + 1 < G) gload(g + 1);
        const uint4 *A = As + buf * TILE_U4;
        const uint4 *B = Bs + buf * TILE_U4;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = as_bf16x8(A[(wm * 64 + i * 32 + li) * ROW_U4 + ks * 2 + lh]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfr[j] = as_bf16x8(B[(wn * 64 + j * 32 + li) * ROW_U4 + ks * 2 + lh]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[i], bfr[j], acc[i][j]);
        }
        if (g + 1 < G) lstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane (column j = lane % 32, half h) register r holds row 8*(r/4) + 4h + r%4
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + li;
            if (n >= N) continue;
            const float bb = a.bias ? bf2f(a.bias[n]) : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M) {
                    uint32_t o = f2bf(acc[i][j][r]);
                    if (a.bias) o = f2bf(bf2f(o) + bb);
                    a.y[(size_t)m * N + n] = (uint16_t)o;
                }
            }
        }
    }
}

int launch_qgemm_mfma(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                      const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits,
                      hipStream_t stream) {
    GemmArgs a;
    a.x = x; a.wq = wq; a.s = s; a.b = b; a.bias = bias; a.y = y;
    a.M = M; a.N = N; a.K = K; a.G = K / BK;
    const int lds = 4 * TILE_U4 * 16;
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    if (bits == 4) {
        static bool cfg4 = false;
        if (!cfg4 && lds > 65536) {
            SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(qgemm_mfma_kernel<4>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds));
            cfg4 = true;
        }
        hipLaunchKernelGGL(qgemm_mfma_kernel<4>, grid, dim3(THREADS), lds, stream, a);
    } else if (bits == 8) {
        static bool cfg8 = false;
        if (!cfg8 && lds > 65536) {
            SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(qgemm_mfma_kernel<8>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds));
            cfg8 = true;
        }
        hipLaunchKernelGGL(qgemm_mfma_kernel<8>, grid, dim3(THREADS), lds, stream, a);
    } else {
        return set_error(SC_EUNSUPPORTED, "qgemm: bits=%d", bits);
    }
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // namespace sc
