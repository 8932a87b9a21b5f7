// Kernel A, generic-K variant: fused dequant-GEMV for M <= 32 rows of x when K is
// a multiple of 64 but not of the 512 (W4) / 256 (W8) that qgemv16.hip needs.
//
// Computes y[m, n] = sum_k x[m, k] * (s[n, g] * q[n, k] + b[n, g]),  g = k / 64,
// for MLX-affine 4/8-bit weights stored [N, K*bits/32] uint32 with bf16 s, b
// [N, K/64] — mx.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits)
// (src/shardcompute/parallel/quantized_linear.py:168-176).
//
// Mapping onto CDNA4:
// * A workgroup owns one tile of 32 output columns (n) and a range of groups
//   along K (split-K across gridDim.y when there are too few tiles to fill
//   256 CUs).  Its waves split that range in chunks of 8 groups.
// * Each wave multiplies with v_mfma_f32_32x32x16_bf16.  Operand B is the
//   weight: lane (n = lane % 32, half h = lane / 32) loads, per group, the 16
//   bytes (W4) / 32 bytes (W8) of row n covering k in [64g + 32h, 64g + 32h + 32),
//   and turns codes into exact bf16 integers in registers (W4: 128 + q via the
//   mantissa OR trick; W8: q).  Four MFMAs consume one group, so every MFMA
//   output P lies inside a single quantization group and is scaled afterwards:
//       acc += s * P + (b - off * s) * xsum[m, g]      (off = 128 for W4, 0 for W8)
//   where xsum[m, g] = sum of x over the group.  Operand A is x (rows m, padded
//   to 32), staged once per workgroup into LDS with each 8-k word permuted to
//   the W4 slot order; rows >= M read row M-1 and their outputs are dropped.
// * No dequantized weight ever reaches memory: HBM traffic is the packed
//   weights, scales, biases, x and y.
// * Waves of the workgroup split K and reduce through LDS; one workgroup covers
//   all of K for its tile (the staged x must fit LDS).
#include "sc_common.h"

namespace sc {

struct SkinnyArgs {
    const uint16_t *x;
    const uint32_t *wq;
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    int M, N, K, G;
    int groups_per_split;
    int vec_sb;           // scales/biases rows are 16-byte aligned and G % 8 == 0
};

// x word (8 consecutive k, natural order) -> W4 operand slot order
// [x0 x4 x1 x5 x2 x6 x3 x7].
__device__ __forceinline__ uint4 permute_w4(uint4 v) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    return o;
}

__device__ __forceinline__ uint32_t comp(uint4 v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ uint32_t bf16_at(uint4 v, int i) {
    uint32_t w = comp(v, i >> 1);
    return (i & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// Row of output D held in register r by lane half h (32x32 MFMA output layout).
__device__ __forceinline__ int dout_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

constexpr int kMaxWaves = 8;

template <int BITS, int NREG>
__global__ void __launch_bounds__(64 * kMaxWaves) qgemv_skinny_kernel(SkinnyArgs a) {
    // Double-buffer the weight registers (prefetch the wave's next chunk during
    // the MFMAs) only where the register budget allows it without spills.
    constexpr bool PREFETCH = (BITS == 4 && NREG <= 4);
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int U4_PER_GROUP_HALF = BITS / 4;     // uint4 loads per lane per group
    constexpr int U4_PER_GROUP_ROW = BITS / 2;      // uint4 per group in a row

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    const int tile = blockIdx.x;
    const int split = 0;
    const int M = a.M, N = a.N;

    const int g_begin = split * a.groups_per_split;
    const int g_end = min(a.G, g_begin + a.groups_per_split);
    const int Gb = g_end - g_begin;
    const int Wb = Gb * 8;            // 8-k words of x in this split
    const int xstride = Wb + 1;       // uint4 per staged row (+1 breaks bank aliasing)

    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    float *xs = reinterpret_cast<float *>(smem + (size_t)M * xstride * 16);

    const int col = lane & 31;
    const int h = lane >> 5;
    const int n = min(tile * 32 + col, N - 1);
    const size_t row_u4 = (size_t)a.K * BITS / 128;   // uint4 per weight row
    const uint4 *wrow = reinterpret_cast<const uint4 *>(a.wq) + (size_t)n * row_u4;
    const uint16_t *srow = a.s + (size_t)n * a.G;
    const uint16_t *brow = a.b + (size_t)n * a.G;

    // ---- first chunk's weights go out before x staging so HBM starts early
    const int nchunks = (Gb + 7) >> 3;
    uint4 wv[8][U4_PER_GROUP_HALF];
    auto load_chunk = [&](int c) {
        const int g0 = g_begin + c * 8;
        const int ng = min(8, g_end - g0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i < ng) {
#pragma unroll
                for (int p = 0; p < U4_PER_GROUP_HALF; ++p)
                    wv[i][p] = wrow[(size_t)(g0 + i) * U4_PER_GROUP_ROW + h * U4_PER_GROUP_HALF + p];
            }
        }
    };
    int c = wave;
    if (c < nchunks) load_chunk(c);

    // ---- stage x[:, split range] (permuted for W4) and per-group sums
    for (int idx = tid; idx < M * Wb; idx += blockDim.x) {
        const int m = idx / Wb;
        const int w = idx - m * Wb;
        uint4 v = *reinterpret_cast<const uint4 *>(a.x + (size_t)m * a.K + (size_t)g_begin * 64 + (size_t)w * 8);
        if (BITS == 4) v = permute_w4(v);
        xl[m * xstride + w] = v;
    }
    __syncthreads();
    for (int idx = tid; idx < M * Gb; idx += blockDim.x) {
        const int m = idx / Gb;
        const int gl = idx - m * Gb;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint4 v = xl[m * xstride + gl * 8 + w];
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += bf2f(bf16_at(v, e));
        }
        xs[m * Gb + gl] = sum;
    }
    __syncthreads();

    float acc[NREG];
#pragma unroll
    for (int r = 0; r < NREG; ++r) acc[r] = 0.f;
    const int arow = min(col, M - 1);
    const uint4 *xa_row = xl + arow * xstride;

    for (; c < nchunks; c += nwaves) {
        const int gl0 = c * 8;
        const int g0 = g_begin + gl0;
        const int ng = min(8, g_end - g0);
        uint32_t sv[8], bv[8];
        if (a.vec_sb && ng == 8) {
            const uint4 s4 = *reinterpret_cast<const uint4 *>(srow + g0);
            const uint4 b4 = *reinterpret_cast<const uint4 *>(brow + g0);
#pragma unroll
            for (int i = 0; i < 8; ++i) { sv[i] = bf16_at(s4, i); bv[i] = bf16_at(b4, i); }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sv[i] = i < ng ? srow[g0 + i] : 0u;
                bv[i] = i < ng ? brow[g0 + i] : 0u;
            }
        }
        uint4 cur[8][U4_PER_GROUP_HALF];
        if (PREFETCH) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int p = 0; p < U4_PER_GROUP_HALF; ++p) cur[i][p] = wv[i][p];
            if (c + nwaves < nchunks) load_chunk(c + nwaves);
        } else {
            if (c != wave) load_chunk(c);
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int p = 0; p < U4_PER_GROUP_HALF; ++p) cur[i][p] = wv[i][p];
        }

#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i < ng) {
                f32x16_t P = {};
                const int wl = (gl0 + i) * 8 + h * 4;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const bf16x8_t A = as_bf16x8(xa_row[wl + t]);
                    bf16x8_t B;
                    if (BITS == 4) {
                        const uint32_t w = comp(cur[i][0], t);
                        B = as_bf16x8(nib_pair(w, 0), nib_pair(w, 4), nib_pair(w, 8), nib_pair(w, 12));
                    } else {
                        const uint4 u = cur[i][t >> 1];
                        const uint32_t w0 = (t & 1) ? u.z : u.x;
                        const uint32_t w1 = (t & 1) ? u.w : u.y;
                        B = as_bf16x8(byte_pair_lo(w0), byte_pair_hi(w0), byte_pair_lo(w1), byte_pair_hi(w1));
                    }
                    P = mfma32x32x16(A, B, P);
                }
                const float sf = bf2f(sv[i]);
                const float bf = bf2f(bv[i]);
                const float cf = (BITS == 4) ? fmaf(-128.f, sf, bf) : bf;
#pragma unroll
                for (int r = 0; r < NREG; ++r) {
                    const int row = min(dout_row(r, h), M - 1);
                    acc[r] = fmaf(sf, P[r], fmaf(cf, xs[row * Gb + gl0 + i], acc[r]));
                }
            }
        }
    }

    // ---- reduce the waves' partial tiles through LDS
    __syncthreads();
    float *red = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int r = 0; r < NREG; ++r) red[(wave * NREG + r) * 64 + lane] = acc[r];
    __syncthreads();
    for (int idx = tid; idx < NREG * 64; idx += blockDim.x) {
        const int r = idx >> 6;
        const int l = idx & 63;
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w) v += red[(w * NREG + r) * 64 + l];
        const int row = dout_row(r, l >> 5);
        const int nn = tile * 32 + (l & 31);
        if (row < M && nn < N) {
            uint32_t o = f2bf(v);
            if (a.bias) o = f2bf(bf2f(o) + bf2f(a.bias[nn]));
            a.y[(size_t)row * N + nn] = (uint16_t)o;
        }
    }
}

// ---------------------------------------------------------------- host launch

struct SkinnyPlan {
    int splits, groups_per_split, waves, lds_bytes;
};

static int lds_need(int M, int gps, int waves, int nreg) {
    const int stage = M * (gps * 8 + 1) * 16 + M * gps * 4;
    const int red = waves * nreg * 64 * 4;
    return stage > red ? stage : red;
}

static int nreg_for(int M) { return M == 1 ? 1 : M <= 8 ? 4 : M <= 16 ? 8 : 16; }

// Waves per workgroup: at least one 8-group chunk per wave; the staged x must fit LDS.
static bool plan_skinny(int M, int N, int G, SkinnyPlan *p) {
    const DeviceInfo &di = device_info();
    (void)N;
    const int nreg = nreg_for(M);
    const int chunks = (G + 7) / 8;
    const int waves = chunks < kMaxWaves ? chunks : kMaxWaves;
    const int lds = lds_need(M, G, waves, nreg);
    if (lds > di.max_lds_per_block) return false;
    p->splits = 1;
    p->groups_per_split = G;
    p->waves = waves;
    p->lds_bytes = lds;
    return true;
}

template <int BITS, int NREG>
static int launch_skinny_t(const SkinnyArgs &a, const SkinnyPlan &p, hipStream_t stream) {
    auto kern = qgemv_skinny_kernel<BITS, NREG>;
    static int configured_lds = 0;
    if (p.lds_bytes > 65536 && p.lds_bytes > configured_lds) {
        SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, p.lds_bytes));
        configured_lds = p.lds_bytes;
    }
    dim3 grid((a.N + 31) / 32, p.splits);
    hipLaunchKernelGGL(kern, grid, dim3(64 * p.waves), p.lds_bytes, stream, a);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_qgemv_skinny(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                        const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits,
                        hipStream_t stream) {
    if (M < 1 || M > 32) return set_error(SC_EINVAL, "qgemv: M=%d outside [1, 32]", M);
    const int G = K / 64;
    SkinnyPlan p;
    if (!plan_skinny(M, N, G, &p))
        return set_error(SC_EUNSUPPORTED, "qgemv: x tile of M=%d K=%d does not fit LDS", M, K);
    SkinnyArgs a;
    a.x = x; a.wq = wq; a.s = s; a.b = b; a.bias = bias; a.y = y;
    a.M = M; a.N = N; a.K = K; a.G = G;
    a.groups_per_split = p.groups_per_split;
    a.vec_sb = ((G % 8) == 0 && ((uintptr_t)s % 16) == 0 && ((uintptr_t)b % 16) == 0) ? 1 : 0;
    const int nreg = nreg_for(M);
#define SC_SKINNY(BITS_, NREG_) \
    if (bits == BITS_ && nreg == NREG_) return launch_skinny_t<BITS_, NREG_>(a, p, stream);
    SC_SKINNY(4, 1) SC_SKINNY(4, 4) SC_SKINNY(4, 8) SC_SKINNY(4, 16)
    SC_SKINNY(8, 1) SC_SKINNY(8, 4) SC_SKINNY(8, 8) SC_SKINNY(8, 16)
#undef SC_SKINNY
    return set_error(SC_EUNSUPPORTED, "qgemv: bits=%d", bits);
}

}  // namespace sc
