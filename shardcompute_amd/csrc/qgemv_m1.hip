// Kernel A at batch 1: persistent dequant-GEMV for one input row, fed by LDS-DMA,
// with the weight items claimed dynamically inside each workgroup.
//
// y[n] = sum_k x[k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// (mx.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits) at M = 1,
//  src/shardcompute/parallel/quantized_linear.py:168-176: every projection and the
//  lm_head of a batch-1 decode step).
//
// The item format, the DMA ring and the MFMA math are those of the M <= 8 kernel
// (qgemv_dma.hip).  What differs, because at batch 1 a launch is short and its
// fixed costs dominate:
// * The input row (for the fused norm also the residual and the norm weight) is
//   fetched by LDS-DMA first, ahead of the weight items, so waiting for it never
//   waits for weights.  Staging and the fused norm take two or three barriers.
// * Waves claim items from a workgroup counter in LDS (the first two per wave are
//   fixed, so the ring fills without waiting on the counter).  A wave the memory
//   system serves late claims fewer items; the waves of a workgroup finish together.
// * Every item writes its 16 column partials to its own LDS slot.  After one
//   barrier each output column is the sum of its tile's items in chunk order, so
//   the result depends on neither the claim order nor timing (bit-reproducible).
#include "dma_util.h"

namespace sc {

struct M1Args {
    const uint16_t *x;       // input row [K] (before the fused norm)
    const uint32_t *wq;
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    int N, K, G;
    int T;                   // 16-row output tiles
    int cpt;                 // items per tile
    unsigned cpt_magic;      // ceil(2^32 / cpt) for cpt > 1: item / cpt == umulhi(item, cpt_magic) for item * cpt < 2^32
    const uint16_t *res;     // PRO_NORM: residual added first (may be null)
    const uint16_t *nw;      // PRO_NORM: norm weight [K]
    float eps;
    uint16_t *h_out;         // PRO_NORM with res: x + res, written by workgroup 0
    uint16_t *x_out;         // PRO_NORM: the normalised row, written by workgroup 0
    int half;                // EPI_SWIGLU: I (gate rows; output width)
    HeadArgmax hd;           // EPI_NONE with hd.key: greedy selection over y
};

namespace {

using namespace dma;
constexpr int M1_MAX_WAVES = 8;
constexpr int M1_PRO_NONE = 0, M1_PRO_NORM = 1;
constexpr int M1_EPI_NONE = 0, M1_EPI_SWIGLU = 1;

__device__ __forceinline__ float sum_bf16x8(uint4 v) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += bf2f(wh(v, e));
    return s;
}

// Greedy selection after the outputs are written (HeadArgmax), by every thread of
// every workgroup: the workgroup's largest key is maxed into *key, then the
// workgroup arrives on *done; the last to arrive turns the key into the token,
// clears the workspace and advances the counters.  Nothing waits on another
// workgroup.  Only the two workspace words are shared within the launch (the
// outputs, ids, tokens and counters are read by later launches), so no cache
// maintenance is needed: each workgroup's max has returned (it is performed at
// the device-wide coherence point of atomics) before its arrival is issued, so the
// arrival that returns P - 1 follows every max, and the exchange issued after it
// reads their combined value.
__device__ __forceinline__ void head_finish(const HeadArgmax &hd, unsigned long long best, unsigned long long *kred) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o);
        best = other > best ? other : best;
    }
    if (lane == 0) kred[wave] = best;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) best = kred[w] > best ? kred[w] : best;
    const unsigned long long was = __hip_atomic_fetch_max(hd.key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(was) : "memory");             // the max has returned before the arrival issues
    const unsigned prev = __hip_atomic_fetch_add(hd.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev != gridDim.x - 1) return;
    const unsigned long long k = __hip_atomic_exchange(hd.key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(hd.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int32_t id = (int32_t)(0xFFFFFFFFu - (uint32_t)k);
    hd.ids[0] = id;
    const long c = hd.step ? hd.step[0] : 0;            // read before the counters advance (step may be one)
    if (hd.tokens && c >= 0 && c < hd.tok_cols) hd.tokens[c] = id;
    for (int i = 0; i < hd.n_counters; ++i) hd.counters[i] += 1;
}

}  // namespace

template <int BITS, int PRO, int EPI>
__global__ void __launch_bounds__(64 * M1_MAX_WAVES) qgemv_m1_kernel(M1Args a) {
    constexpr int SPAN_K = BITS == 4 ? 128 : 64;       // k of one 64-byte span of a row
    constexpr int SPAN_GROUPS = SPAN_K / 64;
    constexpr int SPAN_WORDS = SPAN_K / 8;             // 16-byte x chunks per span
    constexpr int ITEM_K = 4 * SPAN_K;
    constexpr int ITEM_GROUPS = ITEM_K / 64;
    constexpr int MFMAS = BITS == 4 ? 4 : 2;           // per span

    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int ctr;                                 // next item to claim
    __shared__ float red[NORM_THREADS / 64];
    __shared__ unsigned long long kred[M1_MAX_WAVES];   // greedy selection: per-wave keys
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    const int K = a.K, G = a.G, W = K >> 3;
    const int xunits = K >> 9;                          // 1 KB units of one bf16 row

    // LDS: rings | x (W chunks, permuted for W4) | zero block (one item's x chunks) |
    // group sums | per-item partials
    uint8_t *ring = smem + (size_t)wave * RING * SLOT_BYTES;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring;
    uint4 *xl = reinterpret_cast<uint4 *>(smem + (size_t)nwaves * RING * SLOT_BYTES);
    uint4 *xzero = xl + W;
    float *xs = reinterpret_cast<float *>(xzero + 4 * SPAN_WORDS);
    float *part = xs + G;
    // staging: 1 KB unit u lives in ring slot 2 of wave u / S2_UNITS (idle until the
    // ring's first refill, which comes after the staged rows are consumed)
    auto s2_unit = [&](int u) -> uint8_t * {
        return smem + (size_t)(u / S2_UNITS) * RING * SLOT_BYTES + 2 * SLOT_BYTES + (size_t)(u % S2_UNITS) * 1024;
    };
    auto raw = [&](int which, int c) -> uint4 {         // 16-byte chunk c of staged row `which`
        return *reinterpret_cast<const uint4 *>(s2_unit(which * xunits + (c >> 6)) + (c & 63) * 16);
    };

    // ---- 1. input rows by LDS-DMA, before anything else
    auto stage = [&](const uint16_t *src, int which) {
        for (int u = wave; u < xunits; u += nwaves)
            dma16(reinterpret_cast<const uint8_t *>(src) + (size_t)u * 1024 + 16 * lane,
                  (uint32_t)(uintptr_t)s2_unit(which * xunits + u));
    };
    stage(a.x, 0);
    if (PRO == M1_PRO_NORM) {
        if (a.res) stage(a.res, 1);
        stage(a.nw, 2);
    }
    if (tid == 0) ctr = 2 * nwaves;                     // items [0, 2 * nwaves) are fixed below
    if (tid < 4 * SPAN_WORDS) xzero[tid] = make_uint4(0u, 0u, 0u, 0u);

    // ---- 2. this workgroup's tiles and the first two items of this wave
    const int P = gridDim.x;
    const int t_begin = (int)(blockIdx.x * (unsigned)a.T / (unsigned)P);      // T * P < 2^31 (host)
    const int t_end = (int)((blockIdx.x + 1) * (unsigned)a.T / (unsigned)P);
    const int ntl = t_end - t_begin;
    const int cpt = a.cpt;
    const int items = ntl * cpt;
    const size_t row_bytes = (size_t)K * BITS / 8;
    auto wrow = [&](int n0, int r) -> int {             // weight row of row r (0..15) of the tile at column n0
        if (EPI == M1_EPI_SWIGLU) return (r < 8 ? 0 : a.half - 8) + (n0 >> 1) + r;
        return min(n0 + r, a.N - 1);
    };
    // item -> 4 x (4 rows x 256 B, row-rotated) + the 16 rows' scales and biases;
    // past the end the last item is loaded again, so every wave issues the same
    // number of DMA instructions per step and the vmcnt waits stay constant
    auto issue = [&](int item, int slot) {
        const int it = min(item, items - 1);
        const int tl = cpt == 1 ? it : (int)__umulhi((unsigned)it, a.cpt_magic);
        const int ch = it - tl * cpt;
        const int n0 = (t_begin + tl) * 16;
        const uint32_t dst = ring_lds + slot * SLOT_BYTES;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * i + (lane >> 4);
            const int col = ((lane & 15) - r) & 15;
            dma16(reinterpret_cast<const uint8_t *>(a.wq) + (size_t)wrow(n0, r) * row_bytes + col * 16 + ch * 256,
                  dst + i * 1024);
        }
        // scales: lanes 0-15 -> row j; biases: lanes 16-31 -> row j (8 groups, 16 B)
        if (lane < 32)
            dma16((lane < 16 ? a.s : a.b) + (size_t)wrow(n0, lane & 15) * G + ((ch * ITEM_GROUPS) & ~7),
                  dst + SLOT_W);
    };
    const bool has_work = items > 0;
    int held0 = wave, held1 = wave + nwaves, held2 = 0;   // items in ring slots 0, 1, 2
    if (has_work) {
        issue(held0, 0);
        issue(held1, 1);
        wait_vm<2 * DMA_PER_ITEM>();                    // the staging DMA (issued first) is complete
    } else {
        wait_vm<0>();
    }
    __syncthreads();

    // ---- 3. x into LDS (W4: permuted for the span layout) and the 64-element group sums
    auto put_x = [&](int c, uint4 v) {
        xl[c] = BITS == 4 ? perm_w4x(v) : v;
        float g = sum_bf16x8(v);                        // the 8 chunks of a group sit in 8 adjacent lanes
        g = group8_sum(g);
        if ((c & 7) == 0) xs[c >> 3] = g;
    };
    if (PRO == M1_PRO_NORM) {
        // RMSNorm of x (+ res) with the standalone kernel's arithmetic and partition
        // (256 threads, thread t holding chunks t, t + 256, ...; wave sums added in
        // order), so the normalised row has the same bits
        if (tid < NORM_THREADS) {
            float ss = 0.f;
            for (int c = tid; c < W; c += NORM_THREADS) {
                uint4 v = raw(0, c);
                if (a.res) v = add_bf16x8(v, raw(1, c));
                ss = sumsq_bf16x8(ss, v);
            }
            ss = wave_sum(ss);
            if (lane == 0) red[wave] = ss;
        }
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
        const float root = rms_root(tot, K, a.eps);
        for (int c = tid; c < W; c += blockDim.x) {
            uint4 v = raw(0, c);
            if (a.res) {
                v = add_bf16x8(v, raw(1, c));
                if (blockIdx.x == 0 && a.h_out) reinterpret_cast<uint4 *>(a.h_out)[c] = v;
            }
            const uint4 o = norm_bf16x8(v, raw(2, c), root);
            if (blockIdx.x == 0 && a.x_out) reinterpret_cast<uint4 *>(a.x_out)[c] = o;
            put_x(c, o);
        }
    } else {
        for (int c = tid; c < W; c += blockDim.x) put_x(c, raw(0, c));
    }
    __syncthreads();

    // ---- 4. the ring
    // A operand.  Only D rows 0 and 8 (W4) or row 0 (W8) are used, and row i of D
    // depends only on row i of A, so every lane loads x for its k-block, except that
    // W4 uses A-rows 0 and 8 as selectors of the two quantization groups of a span:
    // row 0 must be zero over the second 16 k of each 32-k block (lanes q = 2, 3) and
    // row 8 over the first 16 (q = 0, 1).  Those lanes read a zero block.
    const int j = lane & 15, q = lane >> 4;
    const bool a_zero = BITS == 4 && ((j == 0 && q >= 2) || (j == 8 && q < 2));
    const int epar = BITS == 4 ? (q >> 1) : 0;
    const int xq = BITS == 4 ? 4 * q : 2 * q;
    // bf16 128.0 in both halves, kept in a VGPR for v_and_or_b32
    uint32_t magic = 0x43004300u;
    asm volatile("" : "+v"(magic));
    uint32_t nib_mask = 0x000F000Fu;
    asm volatile("" : "+s"(nib_mask));

    auto compute = [&](int item, int slot) {
        const int ch = cpt == 1 ? 0 : item - (int)__umulhi((unsigned)item, a.cpt_magic) * cpt;
        const uint4 *sl = reinterpret_cast<const uint4 *>(ring + slot * SLOT_BYTES);
        // weights of row j, span t, 16-byte column (4t + q), stored rotated by j
        uint4 wv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) wv[t] = sl[(j >> 2) * 64 + (j & 3) * 16 + ((4 * t + q + j) & 15)];
        const uint4 sv = sl[SLOT_W / 16 + j];
        const uint4 bv = sl[SLOT_W / 16 + 16 + j];
        const int gsub = (ch * ITEM_GROUPS) & 7;        // first group of this item inside the 8 loaded
        const uint4 *xrow = a_zero ? xzero : xl + ch * 4 * SPAN_WORDS;
        uint4 xa[4][MFMAS];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int u = 0; u < MFMAS; ++u) xa[t][u] = xrow[t * SPAN_WORDS + xq + u];
        float xsv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) xsv[t] = xs[(ch * 4 + t) * SPAN_GROUPS + epar];
        // four independent MFMA chains (one per span), interleaved to hide MFMA latency
        f4 P4[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) P4[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < MFMAS; ++u) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                bf16x8_t B;
                if (BITS == 4) {
                    const uint32_t w = wc(wv[t], u);
                    B = as_bf16x8(and_or(w, nib_mask, magic), and_or(w >> 4, nib_mask, magic),
                                  and_or(w >> 8, nib_mask, magic), and_or(w >> 12, nib_mask, magic));
                } else {
                    const uint32_t w0 = wc(wv[t], 2 * u), w1 = wc(wv[t], 2 * u + 1);
                    B = as_bf16x8(byte_pair_lo(w0), byte_pair_hi(w0), byte_pair_lo(w1), byte_pair_hi(w1));
                }
                P4[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[t][u]), B, P4[t], 0, 0, 0);
            }
        }
        // acc = sum_t s * P + (b - off * s) * xsum   (W4 codes carry +128: off = 128)
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int gsel = gsub + t * SPAN_GROUPS + epar;
            const float sf = bf2f(wh(sv, gsel));
            const float bf = bf2f(wh(bv, gsel));
            const float cf = BITS == 4 ? fmaf(-128.f, sf, bf) : bf;
            acc = fmaf(sf, P4[t][0], fmaf(cf, xsv[t], acc));
        }
        if (BITS == 4) acc = xor32_sum(acc);           // D row 0 (lanes 0-15) + D row 8 (lanes 32-47)
        if (q == 0) part[item * 16 + j] = acc;
    };
    auto claim = [&]() -> int {
        int v = 0;
        if (lane == 0) v = atomicAdd(&ctr, 1);
        return __builtin_amdgcn_readfirstlane(v);
    };

    // items claimed by one wave increase, so the first slot holding an item past the
    // end means there is no more work for this wave
    if (has_work) {
        for (;;) {
            held2 = claim();
            issue(held2, 2);
            wait_vm<DMA_PER_ITEM * (RING - 1)>();
            if (held0 >= items) break;
            compute(held0, 0);
            held0 = claim();
            issue(held0, 0);
            wait_vm<DMA_PER_ITEM * (RING - 1)>();
            if (held1 >= items) break;
            compute(held1, 1);
            held1 = claim();
            issue(held1, 1);
            wait_vm<DMA_PER_ITEM * (RING - 1)>();
            if (held2 >= items) break;
            compute(held2, 2);
        }
    }
    wait_vm<0>();                                       // no DMA may land after the workgroup ends
    __syncthreads();

    // ---- 5. per column: the tile's item partials in chunk order, then bf16 (+ bias)
    if (EPI == M1_EPI_SWIGLU) {
        for (int o = tid; o < ntl * 8; o += blockDim.x) {
            const int tl = o >> 3, c = o & 7;
            const float *pp = part + (size_t)tl * cpt * 16;
            float g = 0.f, u = 0.f;
            for (int ch = 0; ch < cpt; ++ch) {
                g += pp[ch * 16 + c];
                u += pp[ch * 16 + 8 + c];
            }
            const int col = (t_begin + tl) * 8 + c;      // gate row col, up row half + col
            uint32_t gb = f2bf(g), ub = f2bf(u);
            if (a.bias) {
                gb = f2bf(bf2f(gb) + bf2f(a.bias[col]));
                ub = f2bf(bf2f(ub) + bf2f(a.bias[a.half + col]));
            }
            a.y[col] = (uint16_t)f2bf(silu_mul_f(bf2f(gb), bf2f(ub)));
        }
    } else {
        const bool head = a.hd.key != nullptr;
        unsigned long long best = 0;
        for (int o = tid; o < ntl * 16; o += blockDim.x) {
            const int tl = o >> 4, c = o & 15;
            const int n = (t_begin + tl) * 16 + c;
            if (n >= a.N) continue;
            const float *pp = part + (size_t)tl * cpt * 16 + c;
            float v = 0.f;
            for (int ch = 0; ch < cpt; ++ch) v += pp[ch * 16];
            uint32_t ob = f2bf(v);
            if (a.bias) ob = f2bf(bf2f(ob) + bf2f(a.bias[n]));
            a.y[n] = (uint16_t)ob;
            if (head) {
                const unsigned long long k = argmax_key(ob, (uint32_t)n);
                best = k > best ? k : best;
            }
        }
        if (head) head_finish(a.hd, best, kred);
    }
}

// ---------------------------------------------------------------- host side

int launch_qgemv_m1(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                    const uint16_t *bias, uint16_t *y, int N, int K, int bits, hipStream_t stream,
                    const DmaFused *fused) {
    if (N <= 0 || K <= 0 || K % 512) return SC_EUNSUPPORTED;   // whole items, 16-byte scale rows
    if (((uintptr_t)x % 16) || ((uintptr_t)wq % 16) || ((uintptr_t)s % 16) || ((uintptr_t)b % 16))
        return SC_EUNSUPPORTED;
    const int pro = fused ? fused->kind : M1_PRO_NONE;
    const int half = fused ? fused->swiglu_half : 0;
    if (pro != M1_PRO_NONE && pro != M1_PRO_NORM) return SC_EUNSUPPORTED;
    if (pro == M1_PRO_NORM && (!fused->norm_weight || ((uintptr_t)fused->norm_weight % 16) ||
                               ((uintptr_t)fused->res % 16)))
        return SC_EUNSUPPORTED;
    if (half > 0 && (half % 8 || N != 2 * half)) return SC_EUNSUPPORTED;
    const HeadArgmax *head = fused ? fused->head : nullptr;
    if (head && (half > 0 || !head->key || !head->done || !head->ids)) return SC_EUNSUPPORTED;
    const DeviceInfo &di = device_info();
    const int item_k = bits == 4 ? 512 : 256;
    const int T = (N + 15) / 16;
    const int CPT = K / item_k;
    const int G = K / 64;
    const int xunits = K / 512;
    const int stage_units = (pro == M1_PRO_NORM ? 3 : 1) * xunits;
    const int lds_cap = di.max_lds_per_block < 160 * 1024 ? di.max_lds_per_block : 160 * 1024;
    const size_t static_lds = 128;                       // counter + norm partials + per-wave keys
    int waves = 0, P = 0;
    size_t lds = 0;
    for (int w = M1_MAX_WAVES; w >= 4; w /= 2) {
        P = di.num_cus;
        while (P > 1 && (long)T * CPT < (long)P * w) P /= 2;   // about one item per wave at least
        const long items_max = (long)((T + P - 1) / P) * CPT;
        lds = (size_t)w * RING * SLOT_BYTES + (size_t)K * 2 + 4 * 16 * 16 + (size_t)G * 4 +
              (size_t)items_max * 16 * 4;
        if (lds + static_lds <= (size_t)lds_cap && stage_units <= w * S2_UNITS) {
            waves = w;
            break;
        }
    }
    if (!waves) return SC_EUNSUPPORTED;
    const long items_max = (long)((T + P - 1) / P) * CPT;
    if ((long)T * P >= (1L << 31) || items_max * CPT >= (1L << 32) / 2) return SC_EUNSUPPORTED;
    M1Args a;
    a.x = x; a.wq = wq; a.s = s; a.b = b; a.bias = bias; a.y = y;
    a.N = N; a.K = K; a.G = G; a.T = T; a.cpt = CPT;
    a.cpt_magic = CPT > 1 ? (unsigned)((0x100000000ULL + (unsigned long long)CPT - 1) / (unsigned long long)CPT) : 0u;
    a.res = fused ? fused->res : nullptr;
    a.nw = fused ? fused->norm_weight : nullptr;
    a.eps = fused ? fused->eps : 0.f;
    a.h_out = fused ? fused->h_out : nullptr;
    a.x_out = fused ? fused->x_out : nullptr;
    a.half = half;
    a.hd = head ? *head : HeadArgmax{};
    auto launch = [&](auto kern, int &configured) -> int {
        if (lds > 65536 && (int)lds > configured) {
            SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            configured = (int)lds;
        }
        hipLaunchKernelGGL(kern, dim3(P), dim3(64 * waves), lds, stream, a);
        SC_HIP_CHECK(hipGetLastError());
        return SC_OK;
    };
    static int cfg[2][2][2] = {};
    const int bi = bits == 4 ? 0 : 1, ei = half > 0 ? 1 : 0;
    int &c = cfg[bi][pro][ei];
#define SC_M1_PICK(B_)                                                                                      \
    do {                                                                                                     \
        if (pro == M1_PRO_NORM && ei) return launch(qgemv_m1_kernel<B_, M1_PRO_NORM, M1_EPI_SWIGLU>, c);     \
        if (pro == M1_PRO_NORM) return launch(qgemv_m1_kernel<B_, M1_PRO_NORM, M1_EPI_NONE>, c);             \
        if (ei) return launch(qgemv_m1_kernel<B_, M1_PRO_NONE, M1_EPI_SWIGLU>, c);                           \
        return launch(qgemv_m1_kernel<B_, M1_PRO_NONE, M1_EPI_NONE>, c);                                     \
    } while (0)
    if (bits == 4) SC_M1_PICK(4);
    SC_M1_PICK(8);
#undef SC_M1_PICK
}

}  // namespace sc
