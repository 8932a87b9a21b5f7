// Kernel A (decode): fused dequant-GEMV for M <= 32 rows of x, 16-column tiles.
//
// y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// (mx.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits),
//  src/shardcompute/parallel/quantized_linear.py:168-176), for MLX-affine
// W4/W8 weights [N, K*bits/32] uint32 with bf16 s, b [N, K/64].
//
// Data path (per wave, per 64-byte "span" of 16 weight rows):
// * Lane (col j = lane % 16, lane-group q = lane / 16) loads 16 contiguous bytes
//   of row n0 + j: one load instruction reads 16 rows x 64 B.  A span is two
//   quantization groups for W4 (128 k) and one for W8 (64 k).
// * Codes become exact bf16 integers in registers (W4: 128 + q by OR-ing the
//   nibble into the mantissa of 128.0; W8: q) and feed
//   v_mfma_f32_16x16x32_bf16 as operand B.  Operand A is x, staged once per
//   workgroup in LDS (8-k words permuted to the W4 slot order).
// * An MFMA sums over all four lane-groups.  For W4, lane-groups 0-1 hold group
//   G and 2-3 hold group G+1 of the span, so A-rows are used as group selectors:
//   A-row v = (parity, m) carries x row m only in the lane-groups of that group
//   parity and zeros elsewhere.  Every output row of the MFMA then lies inside
//   one quantization group and is scaled afterwards:
//       acc += s * P + (b - off * s) * xsum[m, g]    (off = 128 W4, 0 W8)
//   with xsum[m, g] the sum of x over the group (computed at staging).  Rows of
//   x beyond M are zero operands; their outputs are never written.
// * A workgroup stages x for its K range (split) once and owns tiles_per_wg
//   consecutive 16-column tiles; each wave computes whole tiles over that range
//   (chunks in order), streaming its (tile, chunk) items with the next one in
//   flight.  When K is split across workgroups (gridDim.y > 1), each writes an
//   fp32 partial tile and a second kernel sums the partials in split order
//   (deterministic, no cross-workgroup fences).
// Nothing dequantized is written to memory: HBM traffic is packed weights,
// scales, biases, x and y (+ the small partials of split tiles).
#include <mutex>

#include "sc_common.h"
#include "../../include/shardcompute_hip.h"

namespace sc {

struct Gemv16Args {
    const uint16_t *x;
    const uint32_t *wq;
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    float *partials;       // [splits, M, N] fp32 partials (null: the kernel writes y itself)
    int M, N, K, G;
    int spans_per_split;   // multiple of CHUNK_SPANS
    int tiles_per_wg;      // 16-column tiles of one workgroup (its waves take them in turn)
};

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4v;

__device__ __forceinline__ f32x4v mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t u4c(uint4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
__device__ __forceinline__ uint32_t u4h(uint4 v, int i) {   // bf16 element i of 8
    const uint32_t w = u4c(v, i >> 1);
    return (i & 1) ? (w >> 16) : (w & 0xFFFFu);
}

__device__ __forceinline__ uint4 permute_w4_word(uint4 v) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    return o;
}

constexpr int CHUNK_SPANS = 4;
// Waves per workgroup: 16 keeps the M <= 8 variants within 128 VGPRs; the larger
// MROWS variants need the 256-VGPR budget of 8-wave workgroups.
__host__ __device__ constexpr int gemv16_max_waves(int mrows) { return mrows <= 8 ? 16 : 8; }

template <int BITS, int MROWS>
struct G16 {
    static constexpr int SPAN_K = BITS == 4 ? 128 : 64;
    static constexpr int SPAN_GROUPS = SPAN_K / 64;
    static constexpr int SPAN_WORDS = SPAN_K / 8;           // 8-k words of x per span
    static constexpr int MFMA_PER_SET = BITS == 4 ? 4 : 2;  // per span
    static constexpr int CHUNK_GROUPS = CHUNK_SPANS * SPAN_GROUPS;  // 8 (W4) / 4 (W8)
    // virtual A rows: W4 = 2 parities x MP rows, W8 = MROWS rows (at least 16)
    static constexpr int MP = BITS == 4 ? (MROWS < 8 ? 8 : MROWS) : MROWS;
    static constexpr int VROWS = BITS == 4 ? 2 * MP : (MROWS < 16 ? 16 : MROWS);
    static constexpr int NSETS = VROWS / 16;
    __device__ static int parity(int v) { return BITS == 4 ? v / MP : 0; }
    __device__ static int mrow(int v) { return BITS == 4 ? v % MP : v; }
};

template <int BITS, int MROWS>
__global__ void __launch_bounds__(64 * gemv16_max_waves(MROWS)) qgemv16_kernel(Gemv16Args a) {
    using C = G16<BITS, MROWS>;
    extern __shared__ __align__(16) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    const int j = lane & 15;          // column within the tile / A row index
    const int q = lane >> 4;          // lane-group
    const int split = blockIdx.y;
    const int M = a.M, N = a.N;

    const int nspans_total = a.K / C::SPAN_K;
    const int sp_begin = split * a.spans_per_split;
    const int sp_end = min(nspans_total, sp_begin + a.spans_per_split);
    const int nspans = sp_end - sp_begin;
    const int nchunks = nspans / CHUNK_SPANS;     // host guarantees divisibility
    const int Wr = nspans * C::SPAN_WORDS;        // x words staged per row
    const int Gr = nspans * C::SPAN_GROUPS;       // groups in this split
    const int g_begin = sp_begin * C::SPAN_GROUPS;
    const int xstride = Wr + 1;

    // x rows 0..M-1, then row M of zeros: the A operand of a lane that carries no x
    // (a row beyond M, or the other group parity) is read from it, so every x read is
    // unconditional (a conditional read became a branch around each LDS load, which
    // then completed one at a time)
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    float *xs = reinterpret_cast<float *>(smem + (size_t)(M + 1) * xstride * 16);

    // this wave's items: (tile, chunk) for its tiles wave, wave + nwaves, ... of the
    // workgroup, every chunk of the split in order
    const int ntiles = (N + 15) / 16;
    const int tile0 = blockIdx.x * a.tiles_per_wg;
    const int my_tiles = max(0, (min(a.tiles_per_wg, ntiles - tile0) - wave + nwaves - 1) / nwaves);
    const int nitems = my_tiles * nchunks;

    // ---- 1. x words for LDS (first round issued before any weight load)
    // x words held per thread per round: the registers are free before the stream,
    // except in the 16-wave variants (128 VGPRs)
    constexpr int XR = MROWS <= 8 ? 4 : 16;
    const int xwords = M * Wr;
    // word idx is (row idx / Wr, word idx % Wr): the quotient as a multiply-high by
    // ceil(2^32 / Wr), exact for idx * Wr < 2^32 (idx < 32 x 2048, Wr <= 2048); a
    // division by a run-time value would cost tens of instructions per word
    const unsigned wr_magic = (unsigned)((0x100000000ULL + (unsigned)Wr - 1) / (unsigned)Wr);
    auto xrow = [&](int idx) -> int { return Wr == 1 ? idx : (int)__umulhi((unsigned)idx, wr_magic); };
    uint4 xv[XR];
    int round_base = 0;
    auto x_issue = [&](int base) {
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int idx = base + tid + r * blockDim.x;
            if (idx < xwords) {
                const int m = xrow(idx), w = idx - m * Wr;
                xv[r] = *reinterpret_cast<const uint4 *>(a.x + (size_t)m * a.K + (size_t)g_begin * 64 + (size_t)w * 8);
            }
        }
    };
    // stores a round's words and the 64-element group sums of x: the 8 words of a
    // group are 8 adjacent lanes (Wr, the block size and every round base are
    // multiples of 8), each lane sums its word in order, then a 3-step lane tree
    auto x_store = [&](int base) {
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int idx = base + tid + r * blockDim.x;
            const bool in = idx < xwords;
            const int m = xrow(idx), w = idx - m * Wr;
            float g = 0.f;
            if (in) {
                xl[m * xstride + w] = BITS == 4 ? permute_w4_word(xv[r]) : xv[r];
#pragma unroll
                for (int e = 0; e < 8; ++e) g += bf2f(u4h(xv[r], e));
            }
            g = group8_sum(g);                      // lanes converged: the round loop is uniform
            if (in && (w & 7) == 0) xs[m * Gr + (w >> 3)] = g;
        }
    };
    x_issue(0);

    // ---- 2. first chunk of weights + scales/biases
    uint4 wA[CHUNK_SPANS], wB[CHUNK_SPANS];
    uint4 sA, bA, sB, bB;   // W4: 8 groups (uint4); W8: 4 groups in .x/.y
    // item it of this wave: chunk it % nchunks of tile tile0 + wave + nwaves * (it / nchunks)
    auto w_issue = [&](int it, uint4 *w, uint4 &sv, uint4 &bv) {
        const int ti = it / nchunks, c = it - ti * nchunks;
        const int n = min((tile0 + wave + nwaves * ti) * 16 + j, N - 1);
        const uint4 *wrow = reinterpret_cast<const uint4 *>(a.wq) + (size_t)n * ((size_t)a.K * BITS / 128);
        const uint16_t *srow = a.s + (size_t)n * a.G;
        const uint16_t *brow = a.b + (size_t)n * a.G;
        const int sp0 = sp_begin + c * CHUNK_SPANS;
#pragma unroll
        for (int t = 0; t < CHUNK_SPANS; ++t) w[t] = wrow[(size_t)(sp0 + t) * 4 + q];
        const int g0 = sp0 * C::SPAN_GROUPS;
        if (BITS == 4) {
            sv = *reinterpret_cast<const uint4 *>(srow + g0);
            bv = *reinterpret_cast<const uint4 *>(brow + g0);
        } else {
            const uint2 s2 = *reinterpret_cast<const uint2 *>(srow + g0);
            const uint2 b2 = *reinterpret_cast<const uint2 *>(brow + g0);
            sv = make_uint4(s2.x, s2.y, 0u, 0u);
            bv = make_uint4(b2.x, b2.y, 0u, 0u);
        }
    };
    if (nitems > 0) w_issue(0, wA, sA, bA);

    // ---- 3. stage x (remaining rounds wait for everything; only large M*K needs them)
    for (int w = tid; w < xstride; w += blockDim.x) xl[M * xstride + w] = make_uint4(0u, 0u, 0u, 0u);
    x_store(0);
    for (round_base = XR * blockDim.x; round_base < xwords; round_base += XR * blockDim.x) {
        x_issue(round_base);
        x_store(round_base);
    }
    __syncthreads();

    // ---- 4. stream chunks: prefetch the wave's next chunk, then MFMA the current
    f32x4v acc[C::NSETS];
#pragma unroll
    for (int s = 0; s < C::NSETS; ++s) acc[s] = f32x4v{0.f, 0.f, 0.f, 0.f};

    // A-operand row of this lane per set: its x row, or the zero row when it carries
    // no x for this lane-group
    int arow[C::NSETS];
#pragma unroll
    for (int s = 0; s < C::NSETS; ++s) {
        const int v = 16 * s + j;
        const int m = C::mrow(v);
        const bool act = (m < M) && (BITS == 8 || C::parity(v) == (q >> 1));
        arow[s] = act ? m : M;                          // M: the zero row
    }
    // output rows of this lane per set (D row v = 16s + 4q + r)
    int erow[C::NSETS][4];
    int epar[C::NSETS];
#pragma unroll
    for (int s = 0; s < C::NSETS; ++s) {
        epar[s] = C::parity(16 * s + 4 * q);
#pragma unroll
        for (int r = 0; r < 4; ++r) erow[s][r] = min(C::mrow(16 * s + 4 * q + r), M - 1);
    }

    // x operands of a span: every read of the span is issued before its MFMAs, and
    // where registers allow (at most 8 reads a span) the next span's before the
    // current span's MFMAs, so the LDS latency is paid about once per span rather
    // than once per MFMA (the compiler otherwise waited for each read in turn)
    constexpr int XRD = C::NSETS * C::MFMA_PER_SET;          // x reads per span
    constexpr bool XDB = XRD <= 8;                           // next span's reads ahead
    auto x_read = [&](int spl, uint4 (&xa)[XRD]) {
#pragma unroll
        for (int s = 0; s < C::NSETS; ++s)
#pragma unroll
            for (int u = 0; u < C::MFMA_PER_SET; ++u) {
                const int word = spl * C::SPAN_WORDS + (BITS == 4 ? 4 * q + u : 2 * q + u);
                xa[s * C::MFMA_PER_SET + u] = xl[arow[s] * xstride + word];
            }
    };
    // W4 dequant constants in registers the compiler cannot see through: with the
    // literals, (w & mask) | magic became two instructions instead of one v_and_or_b32
    uint32_t nmask = 0x000F000Fu, nmagic = 0x43004300u;
    asm volatile("" : "+s"(nmask));
    asm volatile("" : "+v"(nmagic));
    auto compute_chunk = [&](int cc, const uint4 *w, uint4 sv, uint4 bv) {
        uint4 xa[2][XRD];
        x_read(cc * CHUNK_SPANS, xa[0]);
#pragma unroll
        for (int t = 0; t < CHUNK_SPANS; ++t) {
            const int spl = cc * CHUNK_SPANS + t;     // span index within the split
            const int xb = XDB ? (t & 1) : 0;
            if (XDB && t + 1 < CHUNK_SPANS) x_read(spl + 1, xa[xb ^ 1]);
            if (!XDB && t > 0) x_read(spl, xa[0]);
            const uint4 wv = w[t];
            bf16x8_t B[C::MFMA_PER_SET];
            if (BITS == 4) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t ww = u4c(wv, u);
                    // nib_pair(ww, 0 / 4 / 8 / 12)
                    B[u] = as_bf16x8((ww & nmask) | nmagic, ((ww >> 4) & nmask) | nmagic,
                                     ((ww >> 8) & nmask) | nmagic, ((ww >> 12) & nmask) | nmagic);
                }
            } else {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const uint32_t w0 = u4c(wv, 2 * u), w1 = u4c(wv, 2 * u + 1);
                    B[u] = as_bf16x8(byte_pair_lo(w0), byte_pair_hi(w0), byte_pair_lo(w1), byte_pair_hi(w1));
                }
            }
            f32x4v P[C::NSETS];
#pragma unroll
            for (int s = 0; s < C::NSETS; ++s) {
                P[s] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < C::MFMA_PER_SET; ++u)
                    P[s] = mfma16x16x32(as_bf16x8(xa[xb][s * C::MFMA_PER_SET + u]), B[u], P[s]);
            }
#pragma unroll
            for (int s = 0; s < C::NSETS; ++s) {
                const int gsel = t * C::SPAN_GROUPS + epar[s];   // group within the chunk
                const float sf = bf2f(u4h(sv, gsel));
                const float bf = bf2f(u4h(bv, gsel));
                const float cf = BITS == 4 ? fmaf(-128.f, sf, bf) : bf;
                const int gl = spl * C::SPAN_GROUPS + epar[s];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[s][r] = fmaf(sf, P[s][r], fmaf(cf, xs[erow[s][r] * Gr + gl], acc[s][r]));
            }
        }
    };

    // ---- 5. per finished tile: combine the group parities (final value of (m, column
    // j) per lane: W4 (MROWS <= 8) m = 4q + r in lane-groups q < 2, else m = 16h + 4q + r)
    // and write the tile (or its partial over this split)
    constexpr int NOUT = (BITS == 4) ? (MROWS <= 8 ? 1 : C::NSETS / 2) : C::NSETS;
    auto finish_tile = [&](int ti) {
        f32x4v fin[NOUT];
        if (BITS == 4 && MROWS <= 8) {
#pragma unroll
            for (int r = 0; r < 4; ++r) fin[0][r] = acc[0][r] + __shfl_xor(acc[0][r], 32);
        } else if (BITS == 4) {
#pragma unroll
            for (int h = 0; h < NOUT; ++h) fin[h] = acc[h] + acc[h + NOUT];
        } else {
#pragma unroll
            for (int h = 0; h < NOUT; ++h) fin[h] = acc[h];
        }
        const int nn = (tile0 + wave + nwaves * ti) * 16 + j;
        const bool keepq = (BITS == 4 && MROWS <= 8) ? (q < 2) : true;
        if (nn < N && keepq) {
#pragma unroll
            for (int h = 0; h < NOUT; ++h) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = (BITS == 4 && MROWS <= 8) ? 4 * q + r : 16 * h + 4 * q + r;
                    if (m < M) {
                        const float v = fin[h][r];
                        if (!a.partials) {
                            uint32_t o = f2bf(v);
                            if (a.bias) o = f2bf(bf2f(o) + bf2f(a.bias[nn]));
                            a.y[(size_t)m * N + nn] = (uint16_t)o;
                        } else {
                            a.partials[((size_t)split * M + m) * N + nn] = v;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int s = 0; s < C::NSETS; ++s) acc[s] = f32x4v{0.f, 0.f, 0.f, 0.f};
    };

    // ---- 6. stream the items: the next one in flight while the current one computes
    for (int it = 0; it < nitems; it += 2) {
        if (it + 1 < nitems) w_issue(it + 1, wB, sB, bB);
        compute_chunk(it % nchunks, wA, sA, bA);
        if ((it + 1) % nchunks == 0) finish_tile(it / nchunks);
        if (it + 1 >= nitems) break;
        if (it + 2 < nitems) w_issue(it + 2, wA, sA, bA);
        compute_chunk((it + 1) % nchunks, wB, sB, bB);
        if ((it + 2) % nchunks == 0) finish_tile((it + 1) / nchunks);
    }
}

// Sums split partials in split order, rounds to bf16, adds the bias after rounding.
// With half > 0 the product is gate|up stacked (N = 2 half) and y [M, half] receives
// bf16(silu(gate) * up) of the rounded values, as silu_mul_kernel computes it from
// the bf16 product (parallel/mlp.py:161-162, 241-245).
__global__ void __launch_bounds__(256) qgemv_finalize_kernel(const float *partials, int splits, int M, int N,
                                                              const uint16_t *bias, uint16_t *y, int half) {
    const int64_t total = (int64_t)M * N;
    auto value = [&](int64_t i) -> uint32_t {          // rounded product element i (+ bias)
        float v = 0.f;
        // up to eight loads in flight (a loop of dependent adds issued one load at a
        // time), summed in split order
        int s = 0;
        for (; s + 8 <= splits; s += 8) {
            float p[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) p[u] = partials[(size_t)(s + u) * total + i];
#pragma unroll
            for (int u = 0; u < 8; ++u) v += p[u];
        }
        if (s + 4 <= splits) {
            float p[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) p[u] = partials[(size_t)(s + u) * total + i];
#pragma unroll
            for (int u = 0; u < 4; ++u) v += p[u];
            s += 4;
        }
        for (; s < splits; ++s) v += partials[(size_t)s * total + i];
        uint32_t o = f2bf(v);
        if (bias) o = f2bf(bf2f(o) + bf2f(bias[i % N]));
        return o;
    };
    const int64_t nout = half ? (int64_t)M * half : total;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nout; i += (int64_t)gridDim.x * blockDim.x) {
        if (!half) {
            y[i] = (uint16_t)value(i);
        } else {
            const int64_t m = i / half, c = i - m * half;
            const uint32_t g = value(m * N + c), u = value(m * N + half + c);
            y[i] = (uint16_t)f2bf(silu_mul_f(bf2f(g), bf2f(u)));
        }
    }
}

// ---------------------------------------------------------------- host side

// Split-K partials of the allocation-free entry point (sc_qmm_bf16_noalloc): a
// file-scope device array, one copy per GPU, held until the process ends.  Its
// device address is looked up once per device (hipGetSymbolAddress, with that
// device current) and kept; host code passes only that address to kernels.
// Every entry a split-K launch reads is written by the same launch first, so no
// part of it needs clearing between calls.
static __device__ __align__(256) float scratch[SC_QMM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

static constexpr int kScratchDevices = 64;
static float *g_scratch_ptr[kScratchDevices];
static std::mutex g_scratch_mu;

int qmm_noalloc_scratch(float **out) {
    int dev = 0;
    SC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kScratchDevices) return set_error(SC_EINVAL, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(SC_ELAUNCH, "qmm_noalloc: hipGetSymbolAddress of the scratch array failed on device "
                                         "%d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    *out = g_scratch_ptr[dev];
    return SC_OK;
}

struct Gemv16Plan {
    int splits, spans_per_split, waves, lds, tiles_per_wg, groups;
};

// Work is (tile, split) units of cps chunks each.  Splits: enough units for about
// one per wave of a workgroup per CU, but no fewer than the x slice's LDS allows;
// then ~one workgroup per CU per split, each owning a run of consecutive tiles.
template <int BITS>
static bool plan_gemv16(int M, int N, int K, Gemv16Plan *p) {
    using C = G16<BITS, 8>;
    const int maxw = gemv16_max_waves(M <= 8 ? 8 : 16);
    const DeviceInfo &di = device_info();
    const int tiles = (N + 15) / 16;
    const int chunk_k = CHUNK_SPANS * C::SPAN_K;
    if (K % chunk_k) return false;
    const int nchunks = K / chunk_k;
    const int lds_cap = di.max_lds_per_block < 160 * 1024 ? di.max_lds_per_block : 160 * 1024;
    const int want = (di.num_cus * maxw + tiles - 1) / tiles;     // splits for one unit per wave
    for (int s = want < 1 ? 1 : want; ; ++s) {
        if (s > nchunks) s = nchunks;
        const int cps = (nchunks + s - 1) / s;
        const int real = (nchunks + cps - 1) / cps;
        const int kr = cps * chunk_k;
        const int lds = (M + 1) * (kr / 8 + 1) * 16 + M * (kr / 64) * 4;
        if (lds <= lds_cap) {
            const int groups0 = (di.num_cus + real - 1) / real;
            const int tpw = (tiles + groups0 - 1) / groups0;
            p->splits = real;
            p->spans_per_split = cps * CHUNK_SPANS;
            p->tiles_per_wg = tpw;
            p->groups = (tiles + tpw - 1) / tpw;
            p->waves = tpw < maxw ? tpw : maxw;
            p->lds = lds;
            return true;
        }
        if (s >= nchunks) return false;
    }
}

template <int BITS, int MROWS>
static int launch_gemv16_t(const Gemv16Args &a, const Gemv16Plan &p, hipStream_t stream) {
    auto kern = qgemv16_kernel<BITS, MROWS>;
    static int configured = 0;
    if (p.lds > 65536 && p.lds > configured) {
        SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, p.lds));
        configured = p.lds;
    }
    hipLaunchKernelGGL(kern, dim3(p.groups, p.splits), dim3(64 * p.waves), p.lds, stream, a);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

// Returns SC_EUNSUPPORTED when the shape does not suit this kernel (caller falls back).
// no_alloc: the split-K partials go to the file-scope scratch array (shapes that
// need more than it holds are rejected) instead of the library-owned buffer.
// swiglu_half > 0: the weight is gate|up stacked (N = 2 swiglu_half) and y [M, swiglu_half]
// receives silu(gate) * up, applied by the partials' pass (which then always runs).
// keep (plain products): the partials are left to the caller's pass (keep->splits > 0)
// instead of being summed into y.
int launch_qgemv16(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b, const uint16_t *bias,
                   uint16_t *y, int M, int N, int K, int bits, hipStream_t stream, bool no_alloc, int swiglu_half,
                   SplitKeep *keep) {
    if (M < 1 || M > 32) return SC_EUNSUPPORTED;
    if (swiglu_half && (swiglu_half < 0 || N != 2 * swiglu_half)) return SC_EUNSUPPORTED;
    if (((uintptr_t)s % 16) || ((uintptr_t)b % 16)) return SC_EUNSUPPORTED;
    Gemv16Plan p;
    const bool ok = bits == 4 ? plan_gemv16<4>(M, N, K, &p) : plan_gemv16<8>(M, N, K, &p);
    if (!ok) return SC_EUNSUPPORTED;
    Gemv16Args a;
    a.x = x; a.wq = wq; a.s = s; a.b = b; a.bias = bias; a.y = y; a.partials = nullptr;
    a.M = M; a.N = N; a.K = K; a.G = K / 64; a.spans_per_split = p.spans_per_split;
    a.tiles_per_wg = p.tiles_per_wg;
    const bool with_partials = p.splits > 1 || swiglu_half > 0;
    if (with_partials) {
        const size_t need = (size_t)p.splits * M * N;
        if (no_alloc) {
            constexpr size_t cap = SC_QMM_NOALLOC_SCRATCH_BYTES / sizeof(float);
            // above the array: the caller moves on to a kernel that needs no scratch
            if (need > cap)
                return set_error(SC_EUNSUPPORTED, "qmm_noalloc: M=%d N=%d K=%d needs %zu bytes of split-K scratch, "
                                                  "above the %zu-byte maximum", M, N, K, need * sizeof(float),
                                 (size_t)SC_QMM_NOALLOC_SCRATCH_BYTES);
            const int rc = qmm_noalloc_scratch(&a.partials);
            if (rc) return rc;
        } else {
            SplitKScratch ws;
            const int rc = splitk_scratch(need, 1, &ws);
            if (rc) return rc;
            a.partials = ws.partials;
        }
    }
    int rc;
    const int mrows = M <= 8 ? 8 : M <= 16 ? 16 : 32;
#define SC_G16(B_, R_) if (bits == B_ && mrows == R_) rc = launch_gemv16_t<B_, R_>(a, p, stream); else
    SC_G16(4, 8) SC_G16(4, 16) SC_G16(4, 32) SC_G16(8, 8) SC_G16(8, 16) SC_G16(8, 32)
    return set_error(SC_EUNSUPPORTED, "qgemv16: bits=%d", bits);
#undef SC_G16
    if (rc) return rc;
    if (keep) {
        keep->partials = with_partials ? a.partials : nullptr;
        keep->splits = with_partials ? p.splits : 0;
        if (with_partials && !swiglu_half) return SC_OK;
    }
    if (with_partials) return launch_qmm_finalize(a.partials, p.splits, M, N, bias, y, swiglu_half, stream);
    return SC_OK;
}

int launch_qmm_finalize(const float *partials, int splits, int M, int N, const uint16_t *bias, uint16_t *y, int half,
                        hipStream_t stream) {
    const int64_t total = (int64_t)M * (half ? half : N);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(qgemv_finalize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, partials, splits, M, N,
                       bias, y, half);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // namespace sc
