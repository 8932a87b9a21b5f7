// The MLP activations other than the gated SiLU, and the LayerNorm-style bias of the
// normalisation: the variants ParallelMLP and RMSNorm of the reference accept
// (src/shardcompute/parallel/mlp.py:159-180, 236-250; transformer.py:53-61).
//
//   silu        x / (1 + exp(-x))
//   gelu        x / (1 + exp(-1.702 x))                       (x * sigmoid(1.702 x))
//   gelu_new    0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3)))
//   relu        max(x, 0)   (NaN stays NaN, as mx.maximum)
//   gelu_exact  0.5 x (1 + erf(x / sqrt(2)))
//
// Gated: out[r, i] = bf16(f(gate[r, i]) * up[r, i]) for in = [rows, 2I] (gate columns
// first, up after them, as the fused gate|up product writes them); ungated:
// out[r, i] = bf16(f(in[r, i])).  fp32 arithmetic, each product and sum rounded once
// (no contraction into FMAs), one rounding to bf16 at the end.
#include "sc_common.h"
#include "../../include/shardcompute_hip.h"

namespace sc {

__device__ __forceinline__ float act_f(float x, int kind) {
    switch (kind) {
        case SC_ACT_SILU:
            return __fdiv_rn(x, add_rn(1.f, expf(-x)));
        case SC_ACT_GELU:
            return __fdiv_rn(x, add_rn(1.f, expf(mul_rn(-1.702f, x))));
        case SC_ACT_GELU_NEW: {
            const float x3 = mul_rn(mul_rn(x, x), x);
            const float t = tanhf(mul_rn(0.7978845608028654f, add_rn(x, mul_rn(0.044715f, x3))));
            return mul_rn(mul_rn(0.5f, x), add_rn(1.f, t));
        }
        case SC_ACT_RELU:
            return (x > 0.f || x != x) ? x : 0.f;
        default: {   // SC_ACT_GELU_EXACT
            const float e = erff(mul_rn(x, 0.7071067811865476f));
            return mul_rn(mul_rn(0.5f, x), add_rn(1.f, e));
        }
    }
}

template <bool GATED>
__global__ void __launch_bounds__(256) act_kernel(const uint16_t *__restrict__ in, uint16_t *__restrict__ out,
                                                  long rows, int I, int kind) {
    const int vpr = I >> 3;
    const long nv = rows * vpr;
    for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < nv; idx += (long)gridDim.x * blockDim.x) {
        const long r = idx / vpr;
        const int v = (int)(idx - r * vpr);
        const uint4 a = reinterpret_cast<const uint4 *>(in + (size_t)r * (GATED ? 2 * I : I))[v];
        uint4 u = a;
        if (GATED) u = reinterpret_cast<const uint4 *>(in + (size_t)r * 2 * I + I)[v];
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float y0 = act_f(bfe(a, 2 * e), kind), y1 = act_f(bfe(a, 2 * e + 1), kind);
            if (GATED) {
                y0 = mul_rn(y0, bfe(u, 2 * e));
                y1 = mul_rn(y1, bfe(u, 2 * e + 1));
            }
            o[e] = pack_bf16x2(y0, y1);
        }
        reinterpret_cast<uint4 *>(out + (size_t)r * I)[v] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// out[r, d] = bf16(x[r, d] + bias[d])
__global__ void __launch_bounds__(256) row_bias_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ bias,
                                                       uint16_t *__restrict__ out, long rows, int D) {
    const int vpr = D >> 3;
    const long nv = rows * vpr;
    for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < nv; idx += (long)gridDim.x * blockDim.x) {
        const long r = idx / vpr;
        const int v = (int)(idx - r * vpr);
        const uint4 a = reinterpret_cast<const uint4 *>(x + (size_t)r * D)[v];
        const uint4 b = reinterpret_cast<const uint4 *>(bias)[v];
        reinterpret_cast<uint4 *>(out + (size_t)r * D)[v] = add_bf16x8(a, b);
    }
}

static long grid_for(long nv) {
    long blocks = (nv + 255) / 256;
    const long cap = 8L * device_info().num_cus;
    return blocks > cap ? cap : blocks;
}

}  // namespace sc

using namespace sc;

extern "C" {

int sc_act_bf16(const uint16_t *in, int64_t rows, int64_t I, int kind, int gated, uint16_t *out, void *hip_stream) {
    if (!in || !out) return set_error(SC_EINVAL, "act: null pointer");
    if (kind < SC_ACT_SILU || kind > SC_ACT_GELU_EXACT) return set_error(SC_EINVAL, "act: unknown kind %d", kind);
    if (rows < 0 || I <= 0 || I % 8 || I > (1L << 30)) return set_error(SC_EINVAL, "act: I=%lld must be a multiple of 8",
                                                                         (long long)I);
    if (((uintptr_t)in | (uintptr_t)out) % 16) return set_error(SC_EINVAL, "act: pointers must be 16-byte aligned");
    const size_t in_bytes = (size_t)rows * I * 2 * (gated ? 2 : 1), out_bytes = (size_t)rows * I * 2;
    const uintptr_t a = (uintptr_t)in, o = (uintptr_t)out;
    if (o != a && o < a + in_bytes && a < o + out_bytes)
        return set_error(SC_EINVAL, "act: out overlaps the input (only out == in, ungated, is allowed)");
    if (gated && o == a) return set_error(SC_EINVAL, "act: the gated form cannot run in place");
    if (rows == 0) return SC_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
    const long nv = (long)rows * (I / 8);
    if (gated)
        hipLaunchKernelGGL(act_kernel<true>, dim3((unsigned)grid_for(nv)), dim3(256), 0, st, in, out, (long)rows,
                           (int)I, kind);
    else
        hipLaunchKernelGGL(act_kernel<false>, dim3((unsigned)grid_for(nv)), dim3(256), 0, st, in, out, (long)rows,
                           (int)I, kind);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int sc_add_row_bias_bf16(const uint16_t *x, int64_t rows, int64_t D, const uint16_t *bias, uint16_t *out,
                         void *hip_stream) {
    if (!x || !bias || !out) return set_error(SC_EINVAL, "add_row_bias: null pointer");
    if (rows < 0 || D <= 0 || D % 8 || D > (1L << 30))
        return set_error(SC_EINVAL, "add_row_bias: D=%lld must be a multiple of 8", (long long)D);
    if (((uintptr_t)x | (uintptr_t)bias | (uintptr_t)out) % 16)
        return set_error(SC_EINVAL, "add_row_bias: pointers must be 16-byte aligned");
    if (rows == 0) return SC_OK;
    const long nv = (long)rows * (D / 8);
    hipLaunchKernelGGL(row_bias_kernel, dim3((unsigned)grid_for(nv)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(hip_stream), x, bias, out, (long)rows, (int)D);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // extern "C"
