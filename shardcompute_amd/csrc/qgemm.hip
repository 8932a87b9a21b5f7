// Kernel B: dequant -> bf16 MFMA GEMM for prefill-sized batches.
//
// Same contraction as the decode GEMV (mx.quantized_matmul(..., transpose=True),
// src/shardcompute/parallel/quantized_linear.py:168-176), for larger M:
//     y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
//
// * Workgroup tile 256 (m) x BN (n, 256 or 128), 8 waves in a 2 x 4 grid, each wave
//   128 x BN/4 on v_mfma_f32_32x32x16_bf16 (fp32 accumulators).
// * K advances one quantization group (64) per stage.  LDS holds two stages of the
//   x tile and of the dequantized weight tile (rows of 128 bytes, 16-byte chunks
//   XOR-swizzled by row so the MFMA operand reads are free of bank conflicts).
// * Loads run ahead of use: the packed weights, scales and biases two stages
//   ahead (two register sets, so the stage loop is unrolled by two), the x tile one
//   stage ahead.  During stage g's MFMAs each thread dequantizes its part of stage
//   g+1's weights, a quarter per 16-k step, to bf16(s * q + b) (one fp32 FMA per
//   weight, the reference's dequant) and stores it into the other weight buffer;
//   the x rows of stage g+1 follow after the MFMAs, then one barrier per stage.
// * The grid is ordered so that the workgroups sharing the x rows of one m-tile
//   run on one XCD (workgroups are dealt to the 8 XCDs round robin), which keeps
//   the x tiles in that XCD's L2; the packed weights stream from HBM.
// * The epilogue rounds to bf16 and adds the optional linear bias after that
//   rounding (the reference adds it to the bf16 matmul result,
//   quantized_linear.py:179-180).
#include "sc_common.h"
#include "../../include/shardcompute_hip.h"

namespace sc {

struct GemmArgs {
    const uint16_t *x;
    const uint32_t *wq;
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    int M, N, K, G;
    int ldy;               // y's row stride (N, or wider when this launch covers a column range)
    int mt, nt, tiles;     // m-tiles, n-tiles, real tiles (the grid is padded to a multiple of 8)
    // SwiGLU (swiglu_i = I > 0): the weight stacks gate and up ([2I, K]); the N = 2I
    // product columns are paired, column c of the launch's range holding, per 32-block
    // b and u = c % 32, weight row ic (u < 16, gate) or I + ic (up) with
    // ic = (n_base + c) / 32 * 16 + u % 16; y receives act [M, I] = silu(gate) * up.
    // (The pointers are not offset for a column range; n_base locates it.)
    int swiglu_i, n_base;
    // Split K (grid y = splits): split z takes groups [z gps, z gps + gps) and writes
    // fp32 partials [splits, M, N] (plain products only); gps >= G: no split, y is bf16.
    float *partials;
    int gps;
};

namespace {

constexpr int BM = 256;
constexpr int BK = 64;                    // one quantization group
constexpr int THREADS = 512;
constexpr int ROW_BYTES = BK * 2;         // 128 B of bf16 per tile row
constexpr int XTILE = BM * ROW_BYTES;     // 32 KB
constexpr int XCDS = 8;

template <int BN>
struct Geo {
    static constexpr int WTILE = BN * ROW_BYTES;                 // dequantized weight tile
    static constexpr int STAGE = XTILE + WTILE;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int WN = BN / 4;                            // wave tile width
    static constexpr int NJ = WN / 32;                           // 32-column MFMA blocks per wave
    static constexpr int TPR = THREADS / BN;                     // threads per weight row (2 or 4)
    static constexpr int CPT = BK / TPR;                         // codes per thread and stage (32 or 16)
};

// swizzled byte offset of 16-byte chunk c of tile row r: the MFMA operand reads
// (16 consecutive rows, one chunk) and the row-wise stores (8 chunks of a row, or
// 2-4 rows) then fall on distinct 16-byte bank groups whether the LDS serves 8
// lanes over 32 banks or 16 lanes over 64 banks per cycle
__device__ __forceinline__ uint32_t swz(int r, int c) {
    return (uint32_t)(r * ROW_BYTES + ((c ^ (r & 7) ^ ((r >> 3) & 1)) << 4));
}

template <int BITS, int CPT>
struct WRegs {
    uint32_t w[CPT * BITS / 32];   // this thread's codes of one row and stage
    uint32_t s, b;
};

}  // namespace

template <int BITS, int BN>
__global__ void __launch_bounds__(THREADS) qgemm_mfma_kernel(GemmArgs a) {
    using Gm = Geo<BN>;
    constexpr int CPT = Gm::CPT;
    constexpr int NW = CPT * BITS / 32;          // code words per thread and stage
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int M = a.M, N = a.N, K = a.K;
    const int g0 = (int)blockIdx.y * a.gps;              // this split's first group
    const int G = min(a.G - g0, a.gps);                  // and its stages

    // XCD-aware tile order: workgroup w runs on XCD w % 8; XCD x takes the tiles
    // [x * per, (x + 1) * per) of the m-major order, so its workgroups share x rows
    const int per = (int)(gridDim.x / XCDS);
    const int tile = (int)(blockIdx.x % XCDS) * per + (int)(blockIdx.x / XCDS);
    if (tile >= a.tiles) return;
    const int m0 = (tile / a.nt) * BM;
    const int n0 = (tile % a.nt) * BN;

    // ---- x tile: thread -> chunk (tid & 7) of rows (tid >> 3) + 64 i, i < 4, 16 B each
    // (named registers rather than an array, so that they stay out of scratch)
    const int xr_ = tid >> 3, xc_ = tid & 7;
    const uint16_t *xk = a.x + (size_t)g0 * BK;
    const uint16_t *xs0 = xk + (size_t)min(m0 + xr_, M - 1) * K + xc_ * 8;
    const uint16_t *xs1 = xk + (size_t)min(m0 + xr_ + 64, M - 1) * K + xc_ * 8;
    const uint16_t *xs2 = xk + (size_t)min(m0 + xr_ + 128, M - 1) * K + xc_ * 8;
    const uint16_t *xs3 = xk + (size_t)min(m0 + xr_ + 192, M - 1) * K + xc_ * 8;
    const uint32_t xd = swz(xr_, xc_);      // rows + 64 i land at + 64 * 128 * i (same swizzle)
    uint4 xv0, xv1, xv2, xv3;
    auto load_x = [&](int g) {
        const size_t o = (size_t)g * BK;
        xv0 = *reinterpret_cast<const uint4 *>(xs0 + o);
        xv1 = *reinterpret_cast<const uint4 *>(xs1 + o);
        xv2 = *reinterpret_cast<const uint4 *>(xs2 + o);
        xv3 = *reinterpret_cast<const uint4 *>(xs3 + o);
    };
    auto store_x = [&](int buf) {
        uint8_t *A = smem + buf * Gm::STAGE + xd;
        *reinterpret_cast<uint4 *>(A) = xv0;
        *reinterpret_cast<uint4 *>(A + 64 * ROW_BYTES) = xv1;
        *reinterpret_cast<uint4 *>(A + 128 * ROW_BYTES) = xv2;
        *reinterpret_cast<uint4 *>(A + 192 * ROW_BYTES) = xv3;
    };

    // ---- weights: thread -> (row wr, codes [CPT * wp, CPT * wp + CPT)) of the tile
    const int wr = tid / Gm::TPR, wp = tid % Gm::TPR;
    int wrow = min(n0 + wr, N - 1);
    if (a.swiglu_i) {
        const int c = a.n_base + n0 + wr, u = c & 31;
        const int ic = min((c >> 5) * 16 + (u & 15), a.swiglu_i - 1);
        wrow = u < 16 ? ic : a.swiglu_i + ic;
    }
    const uint8_t *wsrc = reinterpret_cast<const uint8_t *>(a.wq) + (size_t)wrow * ((size_t)K * BITS / 8) +
                          (size_t)g0 * (BK * BITS / 8) + wp * (CPT * BITS / 8);
    const uint16_t *ssrc = a.s + (size_t)wrow * a.G + g0;
    const uint16_t *bsrc = a.b + (size_t)wrow * a.G + g0;
    auto load_w = [&](int g, WRegs<BITS, CPT> &r) {
        const uint8_t *p = wsrc + (size_t)g * (BK * BITS / 8);
        if (NW == 4) {
            const uint4 v = *reinterpret_cast<const uint4 *>(p);
            r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
        } else if (NW == 8) {
            const uint4 v0 = *reinterpret_cast<const uint4 *>(p), v1 = *reinterpret_cast<const uint4 *>(p + 16);
            r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
            r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
        } else {   // NW == 2
            const uint2 v = *reinterpret_cast<const uint2 *>(p);
            r.w[0] = v.x; r.w[1] = v.y;
        }
        r.s = ssrc[g];
        r.b = bsrc[g];
    };
    // The nibble mask lives in an SGPR the compiler cannot see through: with a literal
    // it knows the masked bytes' upper halves are zero and converts bytes 1-3 with a
    // field extract plus a byte-0 conversion, instead of one v_cvt_f32_ubyteN each.
    uint32_t nib = 0x0F0F0F0Fu;
    asm volatile("" : "+s"(nib));
    // dequantize quarter qt (CPT / 4 codes) of a thread's codes into weight buffer buf
    auto store_w = [&](const WRegs<BITS, CPT> &r, int buf, int qt) {
        uint8_t *B = smem + buf * Gm::STAGE + XTILE;
        const float sf = bf2f(r.s), bf = bf2f(r.b);
        constexpr int QC = CPT / 4;                   // codes per quarter: 8 (W4/BN256, W8) or 4
        uint32_t out[QC / 2];
        if (BITS == 4) {
#pragma unroll
            for (int h = 0; h < QC / 8; ++h) {
                const uint32_t w = r.w[qt * (QC / 8) + h];
                const uint32_t lo = w & nib, hi = (w >> 4) & nib;                   // codes 0,2,4,6 / 1,3,5,7
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    out[h * 4 + j] = cvt_pk_bf16(fmaf(sf, ubyte_f32(lo, j), bf), fmaf(sf, ubyte_f32(hi, j), bf));
            }
            if (QC == 4) {   // half a word per quarter
                const uint32_t w = r.w[qt >> 1] >> (16 * (qt & 1));
                const uint32_t lo = w & nib & 0xFFFFu, hi = (w >> 4) & nib & 0xFFFFu;
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    out[j] = cvt_pk_bf16(fmaf(sf, ubyte_f32(lo, j), bf), fmaf(sf, ubyte_f32(hi, j), bf));
            }
        } else {
#pragma unroll
            for (int h = 0; h < QC / 4; ++h) {
                const uint32_t w = r.w[qt * (QC / 4) + h];
                out[h * 2 + 0] = cvt_pk_bf16(fmaf(sf, ubyte_f32(w, 0), bf), fmaf(sf, ubyte_f32(w, 1), bf));
                out[h * 2 + 1] = cvt_pk_bf16(fmaf(sf, ubyte_f32(w, 2), bf), fmaf(sf, ubyte_f32(w, 3), bf));
            }
        }
        // codes [CPT * wp + QC * qt, + QC) are k-chunk (CPT * wp + QC * qt) / 8 of the row
        const int k0 = CPT * wp + QC * qt;
        if (QC == 8) {
            *reinterpret_cast<uint4 *>(B + swz(wr, k0 >> 3)) = make_uint4(out[0], out[1], out[2], out[3]);
        } else {
            *reinterpret_cast<uint2 *>(B + swz(wr, k0 >> 3) + ((k0 & 7) ? 8 : 0)) = make_uint2(out[0], out[1]);
        }
    };

    f32x16_t acc[4][Gm::NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < Gm::NJ; ++j) acc[i][j] = f32x16_t{};

    const int li = lane & 31, lh = lane >> 5;
    // one stage: MFMAs of stage g (buffer buf) with the dequant of the next stage's
    // weights (wnext, into buf ^ 1) interleaved a quarter per 16-k step
    // The operand reads of step ks + 1 are issued before step ks's MFMAs and weight
    // stores (the compiler cannot move LDS reads above LDS stores it cannot prove
    // disjoint), so their latency hides behind the MFMAs.  This takes a second set of
    // operand registers, which W8 with 256-wide tiles does not have to spare; measured
    // on W4 at M = 2048, 256-wide tiles gain 1-5 % and 128-wide ones lose 1-2 %.
    constexpr bool AHEAD = BITS == 4 && BN == 256;
    auto stage = [&](int buf, const WRegs<BITS, CPT> &wnext) {
        const uint8_t *A = smem + buf * Gm::STAGE;
        const uint8_t *Bt = A + XTILE;
        bf16x8_t af[2][4], bfr[2][Gm::NJ];
        auto frag = [&](int ks, int p) {
            const int chunk = ks * 2 + lh;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[p][i] = as_bf16x8(*reinterpret_cast<const uint4 *>(A + swz(wm * 128 + i * 32 + li, chunk)));
#pragma unroll
            for (int j = 0; j < Gm::NJ; ++j)
                bfr[p][j] = as_bf16x8(*reinterpret_cast<const uint4 *>(Bt + swz(wn * Gm::WN + j * 32 + li, chunk)));
        };
        if (AHEAD) frag(0, 0);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int p = AHEAD ? (ks & 1) : 0;
            if (!AHEAD) frag(ks, 0);
            else if (ks + 1 < 4) frag(ks + 1, p ^ 1);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < Gm::NJ; ++j) acc[i][j] = mfma32x32x16(af[p][i], bfr[p][j], acc[i][j]);
            store_w(wnext, buf ^ 1, ks);
        }
    };

    // Every load index is clamped to the last stage and every store is unconditional:
    // past the end they rewrite the buffer not being read, which keeps the loop
    // free of branches between the MFMAs.
    const int gl = G - 1;
    WRegs<BITS, CPT> w0, w1;
    // prologue: stage 0 in LDS, weights of stage 1 in w1, of stage 2 loading into w0
    load_w(0, w0);
    load_x(0);
    load_w(min(1, gl), w1);
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) store_w(w0, 0, qt);
    store_x(0);
    load_w(min(2, gl), w0);
    // With 128-wide tiles the x rows of stage g+1 are loaded before the barrier that
    // starts stage g (XEARLY): when all waves issue their x loads at a stage's start,
    // the issue waits for room in the memory pipeline (about a fifth of a stage,
    // measured), and this way it overlaps the barrier and the rows have a whole stage
    // to arrive.  Measured at M = 2048 (medians of 8 interleaved runs): o and down
    // 2-14 % faster; with 256-wide tiles it was 0-4 % slower, so those keep loading x
    // at the start of the stage that stores it.
    constexpr bool XEARLY = BN == 128;
    if (XEARLY) load_x(min(1, gl));
    __syncthreads();
    // stage g uses buffer g & 1; w1 holds stage g+1 when g is even, w0 when odd
    for (int g = 0; g < G; g += 2) {
        // even stage g: dequant w1 (stage g+1), then load stage g+3 into w1
        if (!XEARLY) load_x(min(g + 1, gl));
        stage(0, w1);
        load_w(min(g + 3, gl), w1);
        store_x(1);
        if (XEARLY) load_x(min(g + 2, gl));
        __syncthreads();
        if (g + 1 < G) {   // odd stage g+1: dequant w0 (stage g+2), then load stage g+4 into w0
            if (!XEARLY) load_x(min(g + 2, gl));
            stage(1, w0);
            load_w(min(g + 4, gl), w0);
            store_x(0);
            if (XEARLY) load_x(min(g + 3, gl));
            __syncthreads();
        }
    }

    // ---- epilogue: lane (column li, half lh) register r holds row 8 * (r / 4) + 4 * lh + r % 4;
    // registers r, r + 1 (rows dm, dm + 1) round to bf16 in one conversion (RNE), and
    // the bias is added to the rounded value and rounded again.  Rows are checked
    // against M only in the last m-tile.
    const int mw = m0 + wm * 128 + 4 * lh;              // row of register 0 of block i = 0
    auto store_tile = [&](auto checked) {
        constexpr bool CHK = decltype(checked)::value;
#pragma unroll
        for (int j = 0; j < Gm::NJ; ++j) {
            const int n = n0 + wn * Gm::WN + j * 32 + li;
            if (n >= N) continue;
            const float bb = a.bias ? bf2f(a.bias[n]) : 0.f;
            uint16_t *yc = a.y + (size_t)mw * a.ldy + n;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    uint32_t o = cvt_pk_bf16(acc[i][j][r], acc[i][j][r + 1]);
                    if (a.bias) o = cvt_pk_bf16(bf2f(o & 0xFFFFu) + bb, bf2f(o >> 16) + bb);
                    const int dm = i * 32 + 8 * (r >> 2) + (r & 3);
                    if (!CHK || mw + dm < M) yc[(size_t)dm * a.ldy] = (uint16_t)o;
                    if (!CHK || mw + dm + 1 < M) yc[(size_t)(dm + 1) * a.ldy] = (uint16_t)(o >> 16);
                }
            }
        }
    };
    // SwiGLU: in each 32-block lanes li < 16 hold gate columns and li >= 16 the up
    // columns of the same ic; after rounding (and the bias) one permlane16 swap gives
    // every lane both halves of its row pair, and lanes li < 16 write the pair's first
    // row, li >= 16 its second: bf16(silu(g) * u) of the rounded g and u, as
    // silu_mul_kernel computes it from the rounded product
    auto store_swiglu = [&](auto checked) {
        constexpr bool CHK = decltype(checked)::value;
        const int I = a.swiglu_i;
        const bool hi = (li & 16) != 0;
#pragma unroll
        for (int j = 0; j < Gm::NJ; ++j) {
            const int c = a.n_base + n0 + wn * Gm::WN + j * 32 + li;
            const int ic = (c >> 5) * 16 + (li & 15);
            const bool ok = ic < I;
            const float bb = a.bias && ok ? bf2f(a.bias[hi ? I + ic : ic]) : 0.f;
            uint16_t *yc = a.y + (size_t)mw * a.ldy + ic;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    uint32_t o = cvt_pk_bf16(acc[i][j][r], acc[i][j][r + 1]);
                    if (a.bias) o = cvt_pk_bf16(bf2f(o & 0xFFFFu) + bb, bf2f(o >> 16) + bb);
                    float gf, uf;                       // (gate pair, up pair) bits
                    swap16(__uint_as_float(o), gf, uf);
                    const uint32_t g = __float_as_uint(gf), u = __float_as_uint(uf);
                    const int sh = hi ? 16 : 0;         // li >= 16: the second row of the pair
                    const float act = silu_mul_f(bf2f((g >> sh) & 0xFFFFu), bf2f((u >> sh) & 0xFFFFu));
                    const int dm = i * 32 + 8 * (r >> 2) + (r & 3) + (hi ? 1 : 0);
                    if (ok && (!CHK || mw + dm < M)) yc[(size_t)dm * a.ldy] = (uint16_t)f2bf(act);
                }
            }
        }
    };
    if (a.partials) {
        // split K: this split's fp32 sums, natural column order, no bias (the split-K
        // pass sums the splits in order, then rounds and adds it)
        float *pz = a.partials + (size_t)blockIdx.y * M * N;
#pragma unroll
        for (int j = 0; j < Gm::NJ; ++j) {
            const int n = n0 + wn * Gm::WN + j * 32 + li;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = mw + i * 32 + 8 * (r >> 2) + (r & 3);
                    if (m < M) pz[(size_t)m * N + n] = acc[i][j][r];
                }
        }
        return;
    }
    if (a.swiglu_i) {
        if (m0 + BM <= M) store_swiglu(std::false_type{});
        else store_swiglu(std::true_type{});
    } else if (m0 + BM <= M) {
        store_tile(std::false_type{});
    } else {
        store_tile(std::true_type{});
    }
}

// One launch over the product's columns [n0, n0 + Nc) with BN-wide tiles.
template <int BITS, int BN>
static int launch_qgemm_cols(const GemmArgs &full, int n0, int Nc, hipStream_t stream) {
    GemmArgs a = full;
    if (full.swiglu_i) {
        a.n_base = n0;
    } else {
        a.wq = full.wq + (size_t)n0 * ((size_t)full.K * BITS / 32);
        a.s = full.s + (size_t)n0 * full.G;
        a.b = full.b + (size_t)n0 * full.G;
        a.bias = full.bias ? full.bias + n0 : nullptr;
        a.y = full.y + n0;
    }
    a.N = Nc;
    a.nt = (Nc + BN - 1) / BN;
    a.tiles = a.mt * a.nt;
    const long blocks = ((long)a.tiles + XCDS - 1) / XCDS * XCDS;
    if (blocks > 0x7FFFFFFFL) return set_error(SC_EINVAL, "qgemm: grid too large");
    if (device_info().max_lds_per_block < Geo<BN>::LDS) return set_error(SC_EUNSUPPORTED, "qgemm: LDS too small");
    auto kern = qgemm_mfma_kernel<BITS, BN>;
    static bool configured = false;
    if (!configured) {
        SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, Geo<BN>::LDS));
        configured = true;
    }
    const int splits = a.partials ? (a.G + a.gps - 1) / a.gps : 1;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks, (unsigned)splits), dim3(THREADS), Geo<BN>::LDS, stream, a);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

template <int BITS>
static int launch_qgemm_t(const GemmArgs &a, hipStream_t stream, bool no_alloc) {
    // The tile width with the shorter estimated time: waves of tiles over the CUs times
    // the cost of one tile, a 128-wide tile costing 0.64 of a 256-wide one (measured
    // on the Llama-3-8B shapes at M = 2048: it reads more LDS per MFMA).  One partial
    // wave of wide tiles beats two waves of narrow ones.
    const int cus = device_info().num_cus;
    const int N = a.N, mt = a.mt;
    const long tiles256 = (long)mt * ((N + 255) / 256);
    // Wide tiles filling at most a quarter of the CUs, over K >= 4096 (a few hundred
    // rows of x): split K so that the tiles times the splits make about one round, each
    // split at least 8 groups; the fp32 partials go through the split-K pass (which
    // applies SwiGLU for a gate|up product, whose columns then stay in their natural
    // order).  Measured on the sweep shapes: at 512 rows, 14336 -> 4096 207 -> 96 us and
    // 5632 -> 2048 84 -> 39 us; with more tiles, or K of 2048, the partials' traffic
    // cost more than the idle CUs (512 x 4096 -> 14336: 91 -> 104 us split in two).
    if (4 * tiles256 <= cus && a.G >= 64) {
        int ks = (int)(cus / tiles256);
        if (ks > a.G / 8) ks = a.G / 8;
        const int gps = (a.G + ks - 1) / ks;
        ks = (a.G + gps - 1) / gps;
        const size_t need = (size_t)ks * a.M * N;
        // without allocation: the allocation-free scratch when the partials fit, else K whole
        if (ks >= 2 && (!no_alloc || need * sizeof(float) <= (size_t)SC_QMM_NOALLOC_SCRATCH_BYTES)) {
            SplitKScratch ws;
            const int rc = no_alloc ? qmm_noalloc_scratch(&ws.partials) : splitk_scratch(need, 1, &ws);
            if (rc) return rc;
            GemmArgs p = a;
            const int half = a.swiglu_i;
            p.swiglu_i = 0;
            p.n_base = 0;
            p.bias = nullptr;
            p.ldy = N;
            p.partials = ws.partials;
            p.gps = gps;
            const int rc2 = launch_qgemm_cols<BITS, 256>(p, 0, N, stream);
            if (rc2) return rc2;
            return launch_qmm_finalize(ws.partials, ks, a.M, N, a.bias, a.y, half, stream);
        }
    }
    const long waves256 = (tiles256 + cus - 1) / cus;
    const long waves128 = ((long)mt * ((N + 127) / 128) + cus - 1) / cus;
    if (!(100 * waves256 <= 64 * waves128)) return launch_qgemm_cols<BITS, 128>(a, 0, N, stream);
    // Wide tiles leaving a partial last round (gate|up at M = 2048: 896 tiles on 256
    // CUs, 3.5 rounds of work in 4): the columns of that round go to a second launch
    // of 128-wide tiles, which fill one round at ~0.64 of a wide tile's time.
    const long r = tiles256 % cus;
    if (r > 0 && tiles256 > cus && N % 256 == 0 && r % mt == 0 && 2 * r <= cus) {
        const int n1 = N - (int)(r / mt) * 256;
        const int rc = launch_qgemm_cols<BITS, 256>(a, 0, n1, stream);
        if (rc) return rc;
        return launch_qgemm_cols<BITS, 128>(a, n1, N - n1, stream);
    }
    return launch_qgemm_cols<BITS, 256>(a, 0, N, stream);
}

// swiglu_half = I > 0: the weight stacks gate and up (N = 2I, I a multiple of 16) and y
// receives act [M, I] = silu(gate) * up (row stride I).  no_alloc: split-K partials only
// in the allocation-free scratch, K kept whole where they do not fit.
int launch_qgemm_mfma(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                      const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits,
                      hipStream_t stream, int swiglu_half, bool no_alloc) {
    if (bits != 4 && bits != 8) return set_error(SC_EUNSUPPORTED, "qgemm: bits=%d", bits);
    if (swiglu_half && (swiglu_half % 16 || N != 2 * swiglu_half)) return SC_EUNSUPPORTED;
    if (K % BK) return set_error(SC_EINVAL, "qgemm: K=%d not a multiple of %d", K, BK);
    if (((uintptr_t)x % 16) || ((uintptr_t)wq % 16))
        return set_error(SC_EINVAL, "qgemm: x and wq must be 16-byte aligned");
    GemmArgs a;
    a.x = x; a.wq = wq; a.s = s; a.b = b; a.bias = bias; a.y = y;
    a.M = M; a.N = N; a.K = K; a.G = K / BK;
    a.ldy = swiglu_half ? swiglu_half : N;
    a.swiglu_i = swiglu_half;
    a.n_base = 0;
    a.mt = (M + BM - 1) / BM;
    a.nt = a.tiles = 0;
    a.partials = nullptr;
    a.gps = a.G;
    return bits == 4 ? launch_qgemm_t<4>(a, stream, no_alloc) : launch_qgemm_t<8>(a, stream, no_alloc);
}

}  // namespace sc
