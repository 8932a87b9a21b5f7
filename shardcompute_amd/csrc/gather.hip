// Kernels C and C': vocab-sharded masked row gathers.
//
// Semantics of QuantizedParallelEmbedding.forward
// (src/shardcompute/parallel/embedding.py:322-356), per token t:
//     in_shard = vocab_start <= id < vocab_start + v_local
//     out[t]   = in_shard ? table[id - vocab_start] : +0.0 row
// C  copies bf16 rows bit for bit (the vocab-parallel bf16 embedding);
// C' dequantizes the selected packed row: bf16(fma(s, q, b)), which equals
// bf16(fp32(s*q) + b) because s*q is exact in fp32.
//
// One wavefront per token, 16-byte vector loads and non-temporal stores (the
// output is written once and never re-read by this kernel); rows of repeated
// ids are served from L2.
#include "sc_common.h"

namespace sc {

template <typename IdT>
__device__ __forceinline__ int64_t load_id(const IdT *ids, int64_t t) { return (int64_t)ids[t]; }

template <typename IdT, bool VEC>
__global__ void __launch_bounds__(256) vocab_gather_kernel(const IdT *ids, int64_t T, const uint16_t *table,
                                                           int64_t v_local, int64_t D, int64_t vocab_start,
                                                           uint16_t *out) {
    const int lane = threadIdx.x & 63;
    const int64_t wave_global = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t t = wave_global; t < T; t += nwaves) {
        const int64_t id = load_id(ids, t);
        const bool in_shard = id >= vocab_start && id < vocab_start + v_local;
        const int64_t local = in_shard ? id - vocab_start : 0;
        if (VEC) {
            const int64_t d16 = D >> 3;
            const uint4 *src = reinterpret_cast<const uint4 *>(table + local * D);
            uint4 *dst = reinterpret_cast<uint4 *>(out + t * D);
            for (int64_t j = lane; j < d16; j += 64) {
                uint4 v = in_shard ? src[j] : make_uint4(0u, 0u, 0u, 0u);
                __builtin_nontemporal_store(v.x, &dst[j].x);
                __builtin_nontemporal_store(v.y, &dst[j].y);
                __builtin_nontemporal_store(v.z, &dst[j].z);
                __builtin_nontemporal_store(v.w, &dst[j].w);
            }
        } else {
            const uint16_t *src = table + local * D;
            uint16_t *dst = out + t * D;
            for (int64_t j = lane; j < D; j += 64) dst[j] = in_shard ? src[j] : (uint16_t)0;
        }
    }
}

template <typename IdT, int BITS>
__global__ void __launch_bounds__(256) qembed_gather_kernel(const IdT *ids, int64_t T, const uint32_t *wq,
                                                            const uint16_t *s, const uint16_t *b,
                                                            int64_t v_local, int64_t D, int64_t vocab_start,
                                                            uint16_t *out) {
    constexpr int WORDS8 = BITS / 4;   // words holding 8 codes
    const int lane = threadIdx.x & 63;
    const int64_t wave_global = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    const int64_t G = D / 64;
    const int64_t row_words = D * BITS / 32;
    for (int64_t t = wave_global; t < T; t += nwaves) {
        const int64_t id = load_id(ids, t);
        const bool in_shard = id >= vocab_start && id < vocab_start + v_local;
        const int64_t local = in_shard ? id - vocab_start : 0;
        const uint32_t *wr = wq + local * row_words;
        uint4 *dst = reinterpret_cast<uint4 *>(out + t * D);
        for (int64_t j = lane; j < D / 8; j += 64) {   // 8 output values per step
            uint4 o = make_uint4(0u, 0u, 0u, 0u);
            if (in_shard) {
                const int64_t g = (j * 8) / 64;
                const float sf = bf2f(s[local * G + g]);
                const float bf = bf2f(b[local * G + g]);
                float v[8];
                if (BITS == 4) {
                    const uint32_t w = wr[j];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = fmaf(sf, (float)((w >> (4 * e)) & 0xFu), bf);
                } else {
                    const uint32_t w0 = wr[2 * j], w1 = wr[2 * j + 1];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = fmaf(sf, (float)((w0 >> (8 * e)) & 0xFFu), bf);
                        v[4 + e] = fmaf(sf, (float)((w1 >> (8 * e)) & 0xFFu), bf);
                    }
                }
                o = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                               pack_bf16x2(v[6], v[7]));
            }
            (void)WORDS8;
            dst[j] = o;
        }
    }
}

static int gather_grid(int64_t T) {
    const int64_t waves = T < 1 ? 1 : T;
    int64_t blocks = (waves + 3) / 4;
    const int64_t cap = (int64_t)device_info().num_cus * 16;
    if (blocks > cap) blocks = cap;
    return (int)blocks;
}

int launch_vocab_gather(const void *ids, int ids_is_int64, int64_t T, const uint16_t *table, int64_t v_local,
                        int64_t D, int64_t vocab_start, uint16_t *out, hipStream_t stream) {
    const bool vec = (D % 8 == 0) && ((uintptr_t)table % 16 == 0) && ((uintptr_t)out % 16 == 0);
    const dim3 grid(gather_grid(T)), block(256);
#define SC_GATHER(IDT)                                                                                     \
    if (vec)                                                                                               \
        hipLaunchKernelGGL((vocab_gather_kernel<IDT, true>), grid, block, 0, stream, (const IDT *)ids, T, \
                           table, v_local, D, vocab_start, out);                                           \
    else                                                                                                   \
        hipLaunchKernelGGL((vocab_gather_kernel<IDT, false>), grid, block, 0, stream, (const IDT *)ids, T,\
                           table, v_local, D, vocab_start, out);
    if (ids_is_int64) { SC_GATHER(int64_t) } else { SC_GATHER(int32_t) }
#undef SC_GATHER
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_qembed_gather(const void *ids, int ids_is_int64, int64_t T, const uint32_t *wq, const uint16_t *s,
                         const uint16_t *b, int64_t v_local, int64_t D, int64_t vocab_start, int bits,
                         uint16_t *out, hipStream_t stream) {
    const dim3 grid(gather_grid(T)), block(256);
#define SC_QG(IDT, BITS_)                                                                                  \
    hipLaunchKernelGGL((qembed_gather_kernel<IDT, BITS_>), grid, block, 0, stream, (const IDT *)ids, T, wq,\
                       s, b, v_local, D, vocab_start, out);
    if (ids_is_int64) {
        if (bits == 4) { SC_QG(int64_t, 4) } else { SC_QG(int64_t, 8) }
    } else {
        if (bits == 4) { SC_QG(int32_t, 4) } else { SC_QG(int32_t, 8) }
    }
#undef SC_QG
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // namespace sc
