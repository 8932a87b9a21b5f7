// Kernel C: the middle band of the quantized product, 9 <= M <= 256 rows of x.
//
// y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// (mx.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits),
//  src/shardcompute/parallel/quantized_linear.py:168-176), for batched decode
// (16-32 rows), short prefill chunks and the vocab-sharded lm_head over a batch of
// last positions (transformer.py:466-475).  Here the product is bandwidth-bound or
// close to the ridge (4 M flops per W4 weight byte), so the kernel is built around
// the weight stream rather than around MFMA tiles:
//
// * A workgroup owns BN = 32 x (consumer waves) weight rows over a K range (one K
//   split) and all M rows of x (MT blocks of 32).  Each consumer wave owns 32 weight
//   rows: the B operand of v_mfma_f32_32x32x16_bf16, shared by the MT x blocks (the A
//   operands), so every weight is dequantized once per workgroup.
// * Four producer waves issue every LDS-DMA (global_load_lds_dwordx4) and do nothing
//   else, so an issue that waits for room in the CU's memory queue stalls only them.
//   (Measured on the 64-row lm_head: the stream alone, with the consumers idle, takes
//   34 us with four producers and 46 us with two; the consumers' arithmetic alone
//   takes 49 us, so the arithmetic, not the stream, now bounds the kernel.)
// * K advances one quantization group (64) per stage; one barrier per stage.  Three
//   LDS rings, each fed ahead of use:
//     x       one stage (32 MT rows x 128 B) per slot, NX slots;
//     codes   one "item" of IG groups (128 B of every weight row: 4 groups W4, 2 W8)
//             per slot, 3 slots, loaded in IG pieces with the x stages (a weight row's
//             bytes arrive as whole 128-byte lines, not as 32-byte pieces of lines);
//     s, b    the 8 groups' scales and biases of the BN rows, 2 block slots.
//   Every stage's DMA list has the same length per producer, so each producer waits
//   for its part of stage g with one vmcnt immediate; the barrier then publishes the
//   stage and frees the slots the previous stage read.
// * Dequant in registers.  Above 32 rows: bf16(s q + b), one fp32 FMA per weight (the
//   GEMM's rule).  Up to 32 rows (one x block): the decode GEMVs' rule, exact codes on
//   MFMA and the group's scale and bias applied to its fp32 sums (s P + b S), so that
//   a decode batch rounds as a single sequence does.  The k order inside a group is
//   permuted so that a lane's codes of the 4 MFMA k-steps are one 16-byte LDS read
//   (W4): lane half h, step ks holds k = 32 h + 8 ks + e; x rows use the same order
//   (16-byte chunk 4 h + ks).
// * Rows are XOR-swizzled in 16-byte chunks (x by row, codes by row / 2), so the
//   operand reads are free of LDS bank conflicts; the DMA writes lanes in order, so
//   each lane loads the chunk that belongs at its position.
// * With one K split the tile is rounded to bf16 and written (bias after rounding);
//   with several, each split writes fp32 partials and the split-K pass sums them in
//   split order (deterministic).
#include "dma_util.h"
#include "../../include/shardcompute_hip.h"

namespace sc {

struct BandArgs {
    const uint16_t *x;
    const uint8_t *wq;      // packed codes, rows of K * bits / 8 bytes
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    float *partials;        // [ksplit, M, N] fp32, or null: y is written directly
    int M, N, K, G;
    int gps;                // groups per K split (a multiple of 8)
};

namespace band {

using namespace dma;

constexpr int NP = 4;                                  // producer waves
constexpr int LDS_CAP = 152 * 1024;

// x ring slots that fit beside the code and scale/bias rings, capped where the code
// ring's refill would overtake its readers (x runs NX - 1 stages ahead; a code item is
// loaded over the IG stages before its first use, into the slot two items back:
// NX - 1 < IG + 2)
__host__ __device__ constexpr int band_nx(int bits, int mt, int nw) {
    return ((LDS_CAP - 3 * (32 * nw * 128) - 2 * (1024 * nw)) / (mt * 4096)) < (bits == 4 ? 6 : 4)
               ? ((LDS_CAP - 3 * (32 * nw * 128) - 2 * (1024 * nw)) / (mt * 4096))
               : (bits == 4 ? 6 : 4);
}

template <int BITS, int MT, int NW>
struct Geo {
    static constexpr int BN = 32 * NW;                 // weight rows per workgroup
    static constexpr int XB = MT * 32 * 128;           // x stage: 32 MT rows x 64 bf16
    static constexpr int WROW = BITS == 4 ? 32 : 64;   // bytes of one weight row per group
    static constexpr int IG = 128 / WROW;              // groups per code item
    static constexpr int WIB = BN * 128;               // code item bytes
    static constexpr int SBB = 2 * BN * 16;            // scales then biases, 8 groups of BN rows
    static constexpr int NX = band_nx(BITS, MT, NW);   // x ring slots
    static constexpr int LX = NX - 1;                  // stages the x DMA runs ahead
    static constexpr int O_W = NX * XB;                // LDS: x ring, code ring, s/b slots
    static constexpr int O_SB = O_W + 3 * WIB;
    static constexpr int LDS = O_SB + 2 * SBB;
    static constexpr int XI = XB / 1024;               // DMA instructions per stage: x,
    static constexpr int WPI = WIB / 1024 / IG;        // a piece of a code item,
    static constexpr int TI = WPI + 1 + XI;            // one scale/bias instruction
    static constexpr int DP = (TI + NP - 1) / NP;      // per producer: DP or DP - 1
    static constexpr int NFULL = TI % NP == 0 ? NP : TI % NP;   // producers issuing DP
    static constexpr int THREADS = 64 * (NW + NP);
    static_assert(NX >= 2 && LX < IG + 2, "x ring");
    static_assert(LDS <= LDS_CAP, "LDS");
    static_assert((LX - 1) * DP < 64, "vmcnt range");
};

}  // namespace band

using namespace band;

// The LDS holds one workgroup per CU, so (NW + NP) / 4 waves share a SIMD.  With 8 x
// blocks the compiler, left to aim for more waves, keeps the accumulators and x
// operands in fewer registers and serialises each MFMA behind its LDS read; told the
// real occupancy it prefetches them (160 rows: 38.5 -> 32.3 us on a 4096 x 6144
// product).  The smaller blocks measured no faster with it.
template <int BITS, int MT, int NW>
__global__ void __launch_bounds__(64 * (NW + NP))
__attribute__((amdgpu_waves_per_eu((NW + NP + 3) / 4, MT >= 8 ? (NW + NP + 3) / 4 : 8)))
qgemm_band_kernel(BandArgs a) {
    using C = Geo<BITS, MT, NW>;
    constexpr int NX = C::NX, LX = C::LX, IG = C::IG;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, N = a.N;
    const int n0 = blockIdx.x * C::BN;
    const int split = blockIdx.y;
    const int g0 = split * a.gps;
    const int ng = min(a.G - g0, a.gps);               // groups of this split, a multiple of 8
    const int nb = ng >> 3;                            // scale/bias blocks
    const int ni = ng / IG;                            // code items
    const size_t row_bytes = (size_t)a.K * BITS / 8;

    if (wave >= NW) {
        // ================================================================ producers
        // Stage t's list: the code piece (t - 1) % IG of item (t - 1) / IG + 1 (item j's
        // last piece rides with stage IG j, so waiting for stage IG j's x covers it),
        // the scale/bias instruction t % 8 of block t / 8 + 1 (repeats of the last
        // instruction when the block has fewer than 8; block b's last rides with stage
        // 8b - 1), then the x stage.  Instruction i goes to producer i % NP.  Indices
        // past the split are clamped: the reloads rewrite slots nobody reads any more
        // (or the same bytes).
        const int pw = wave - NW;
        const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
        const uint8_t *xbase = reinterpret_cast<const uint8_t *>(a.x) + (size_t)g0 * 128;
        const uint8_t *wbase = a.wq + (size_t)n0 * row_bytes + (size_t)g0 * C::WROW;
        // per-lane offsets, the same for every stage
        // x instruction q: rows 8q + lane / 8, position p = lane % 8 holds chunk p ^ swz(row)
        auto xoff = [&](int q) -> uint32_t {
            const int xr = 8 * q + (lane >> 3);
            const int c = (lane & 7) ^ (xr & 7) ^ ((xr >> 3) & 1);
            return (uint32_t)((min(xr, M - 1) * a.K + 8 * c) * 2);
        };
        // code instruction q of an item: rows 8q + lane / 8, position p holds chunk p ^ (row / 2 % 8)
        auto woff = [&](int q) -> uint32_t {
            const int wr = 8 * q + (lane >> 3);
            const int c = (lane & 7) ^ ((wr >> 1) & 7);
            return (uint32_t)((size_t)(min(n0 + wr, N - 1) - n0) * row_bytes + 16 * c);
        };
        auto issue_sb = [&](int u, int blk) __attribute__((always_inline)) {
            // chunks [64 u, 64 u + 64) of [scales BN | biases BN]: instructions u < NW / 2
            // are scales, the rest biases
            const bool is_b = u >= NW / 2;
            const int row = min(n0 + 64 * u + lane - (is_b ? C::BN : 0), N - 1) - n0;
            const uint8_t *base =
                reinterpret_cast<const uint8_t *>((is_b ? a.b : a.s) + (size_t)n0 * a.G + g0 + 8 * blk);
            dma16s(base, (uint32_t)(row * a.G * 2), lds0 + C::O_SB + (blk & 1) * C::SBB + 1024 * u);
        };
        auto issue_w = [&](int item, int q) __attribute__((always_inline)) {
            // instruction q of code item `item` (clamped to the split) into its slot
            const int ic = min(item, ni - 1);
            dma16s(wbase + (size_t)ic * 128, woff(q), lds0 + C::O_W + (item % 3) * C::WIB + 1024 * q);
        };
        auto issue = [&](int t) __attribute__((always_inline)) {
            const int tc = min(t, ng - 1);
            const int item = (t + IG - 1) / IG, piece = (t + IG - 1) % IG;     // (t - 1) / IG + 1, (t - 1) % IG
            const uint32_t xs = lds0 + (t % NX) * C::XB;
#pragma unroll
            for (int r = 0; r < C::DP; ++r) {
                const int i = pw + r * NP;
                if (i < C::WPI) issue_w(item, piece * C::WPI + i);
                else if (i == C::WPI) issue_sb(min(t & 7, NW - 1), min((t >> 3) + 1, nb - 1));
                else if (i < C::TI) dma16s(xbase + (size_t)tc * 128, xoff(i - C::WPI - 1), xs + 1024 * (i - C::WPI - 1));
            }
        };
        // prologue: code item 0 (all but its last piece, which rides with stage 0),
        // scale/bias block 0, stages 0 .. LX - 1
        for (int q = pw; q < (IG - 1) * C::WPI; q += NP) issue_w(0, q);
        for (int u = pw; u < NW; u += NP) issue_sb(u, 0);
        for (int t = 0; t < LX; ++t) issue(t);
        for (int g = 0; g < ng; ++g) {
            // this producer's part of stage g (and everything it issued before) landed
            if (pw < C::NFULL) wait_vm<(LX - 1) * C::DP>();
            else wait_vm<(LX - 1) * (C::DP - 1)>();
            __syncthreads();                                // stage g visible; slots of g - 1 free
            issue(g + LX);
        }
        wait_vm<0>();                                       // no DMA may land after the workgroup ends
        return;
    }

    // ==================================================================== consumers
    const int li = lane & 31, h = lane >> 5;
    const int rr = 32 * wave + li;                     // this lane's weight row in the tile
    uint32_t nib = 0x0F0F0F0Fu;                        // opaque: one v_cvt_f32_ubyteN per code
    asm volatile("" : "+s"(nib));
    uint32_t nib16 = 0x000F000Fu, magic = 0x43004300u; // opaque: one v_and_or_b32 per code pair
    asm volatile("" : "+s"(nib16));
    asm volatile("" : "+v"(magic));
    f32x16_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x16_t{};

    // x operand (row 32 i + li, 16-byte chunk 4 h + ks) of a stage
    auto xoff = [&](int i, int ks) -> uint32_t {
        const int r = 32 * i + li;
        return (uint32_t)(r * 128 + ((((4 * h + ks) ^ (r & 7) ^ ((r >> 3) & 1))) << 4));
    };
    const int wsw = (rr >> 1) & 7;                     // this row's chunk swizzle in a code item
    auto compute = [&](int xslot, int wslot, int gi, int j, uint4 sv, uint4 bv) __attribute__((always_inline)) {
        const uint8_t *xs = smem + xslot * C::XB;
        const uint8_t *ws = smem + C::O_W + wslot * C::WIB + rr * 128;
        const float sf = bf2f(wh(sv, j)), bf = bf2f(wh(bv, j));
        uint4 wv0, wv1;
        if (BITS == 4) {       // group gi = chunks 2 gi, 2 gi + 1; this lane's half h
            wv0 = *reinterpret_cast<const uint4 *>(ws + 16 * ((2 * gi + h) ^ wsw));
            wv1 = wv0;
        } else {               // group gi = chunks 4 gi .. 4 gi + 3; this lane's two
            wv0 = *reinterpret_cast<const uint4 *>(ws + 16 * ((4 * gi + 2 * h) ^ wsw));
            wv1 = *reinterpret_cast<const uint4 *>(ws + 16 * ((4 * gi + 2 * h + 1) ^ wsw));
        }
        if constexpr (MT == 1) {
            // Up to 32 rows: the decode GEMVs' rule (qgemv_m1_kernel, qgemv16_kernel),
            // so a batch computes as one sequence does: the MFMAs take the exact codes
            // (W4: 128 + q in bf16, slots [q0 q4 q1 q5 q2 q6 q3 q7], x permuted alike;
            // W8: q), a second MFMA chain with all-ones weights sums the group's x, and
            // y += s * P + (b - 128 s) * S (W8: b * S) in fp32.
            const uint32_t ones = 0x3F803F80u;
            const bf16x8_t B1 = as_bf16x8(ones, ones, ones, ones);
            f32x16_t P = f32x16_t{}, S = f32x16_t{};
            uint4 xn = *reinterpret_cast<const uint4 *>(xs + xoff(0, 0));
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                uint4 xv = xn;
                if (ks + 1 < 4) xn = *reinterpret_cast<const uint4 *>(xs + xoff(0, ks + 1));
                bf16x8_t B;
                if (BITS == 4) {
                    xv = perm_w4x(xv);
                    const uint32_t w = wc(wv0, ks);
                    B = as_bf16x8(and_or(w, nib16, magic), and_or(w >> 4, nib16, magic),
                                  and_or(w >> 8, nib16, magic), and_or(w >> 12, nib16, magic));
                } else {
                    const uint4 v = ks < 2 ? wv0 : wv1;
                    const uint32_t w0 = wc(v, 2 * (ks & 1)), w1 = wc(v, 2 * (ks & 1) + 1);
                    B = as_bf16x8(byte_pair_lo(w0), byte_pair_hi(w0), byte_pair_lo(w1), byte_pair_hi(w1));
                }
                P = mfma32x32x16(as_bf16x8(xv), B, P);
                S = mfma32x32x16(as_bf16x8(xv), B1, S);
            }
            const float cf = BITS == 4 ? fmaf(-128.f, sf, bf) : bf;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[0][r] = fmaf(sf, P[r], fmaf(cf, S[r], acc[0][r]));
            return;
        }
        // x operands one k-step ahead of the MFMAs that use them
        uint4 xa[2][MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) xa[0][i] = *reinterpret_cast<const uint4 *>(xs + xoff(i, 0));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks + 1 < 4) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
                    xa[(ks + 1) & 1][i] = *reinterpret_cast<const uint4 *>(xs + xoff(i, ks + 1));
            }
            bf16x8_t B;
            if (BITS == 4) {
                const uint32_t w = wc(wv0, ks);
                const uint32_t lo = w & nib, hi = (w >> 4) & nib;       // codes 0 2 4 6 / 1 3 5 7
                B = as_bf16x8(cvt_pk_bf16(fmaf(sf, ubyte_f32(lo, 0), bf), fmaf(sf, ubyte_f32(hi, 0), bf)),
                              cvt_pk_bf16(fmaf(sf, ubyte_f32(lo, 1), bf), fmaf(sf, ubyte_f32(hi, 1), bf)),
                              cvt_pk_bf16(fmaf(sf, ubyte_f32(lo, 2), bf), fmaf(sf, ubyte_f32(hi, 2), bf)),
                              cvt_pk_bf16(fmaf(sf, ubyte_f32(lo, 3), bf), fmaf(sf, ubyte_f32(hi, 3), bf)));
            } else {
                const uint4 v = ks < 2 ? wv0 : wv1;
                const uint32_t w0 = wc(v, 2 * (ks & 1)), w1 = wc(v, 2 * (ks & 1) + 1);
                B = as_bf16x8(cvt_pk_bf16(fmaf(sf, ubyte_f32(w0, 0), bf), fmaf(sf, ubyte_f32(w0, 1), bf)),
                              cvt_pk_bf16(fmaf(sf, ubyte_f32(w0, 2), bf), fmaf(sf, ubyte_f32(w0, 3), bf)),
                              cvt_pk_bf16(fmaf(sf, ubyte_f32(w1, 0), bf), fmaf(sf, ubyte_f32(w1, 1), bf)),
                              cvt_pk_bf16(fmaf(sf, ubyte_f32(w1, 2), bf), fmaf(sf, ubyte_f32(w1, 3), bf)));
            }
#pragma unroll
            for (int i = 0; i < MT; ++i) acc[i] = mfma32x32x16(as_bf16x8(xa[ks & 1][i]), B, acc[i]);
        }
    };

    int xslot = 0, wslot = 0;
    for (int bk = 0; bk < nb; ++bk) {
        uint4 sv = make_uint4(0u, 0u, 0u, 0u), bv = sv;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            __syncthreads();                          // stage 8 bk + j landed
            if (j == 0) {
                const uint8_t *sb = smem + C::O_SB + (bk & 1) * C::SBB;
                sv = *reinterpret_cast<const uint4 *>(sb + 16 * rr);
                bv = *reinterpret_cast<const uint4 *>(sb + 16 * (C::BN + rr));
            }
            compute(xslot, wslot, j % IG, j, sv, bv);
            xslot = xslot + 1 == NX ? 0 : xslot + 1;
            if (j % IG == IG - 1) wslot = wslot + 1 == 3 ? 0 : wslot + 1;
        }
    }

    // ---- epilogue: lane (column li, half h) register r holds row 8 (r / 4) + 4 h + r % 4
    // of each 32-row block
    const int n = n0 + rr;
    if (n < N) {
        const float bb = (!a.partials && a.bias) ? bf2f(a.bias[n]) : 0.f;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < M) {
                    if (a.partials) {
                        a.partials[((size_t)split * M + m) * N + n] = acc[i][r];
                    } else {
                        uint32_t o = f2bf(acc[i][r]);
                        if (a.bias) o = f2bf(bf2f(o) + bb);
                        a.y[(size_t)m * N + n] = (uint16_t)o;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------- host side

template <int BITS, int MT, int NW>
static int launch_band_t(const BandArgs &a, int tiles, int ksplit, hipStream_t stream) {
    using C = Geo<BITS, MT, NW>;
    if (device_info().max_lds_per_block < C::LDS) return set_error(SC_EUNSUPPORTED, "qgemm_band: LDS too small");
    auto kern = qgemm_band_kernel<BITS, MT, NW>;
    static bool configured = false;
    if (!configured) {
        SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS));
        configured = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)ksplit), dim3(C::THREADS), C::LDS, stream, a);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

// 8 consumer waves (256 rows per workgroup) up to 64 rows of x; 4 above (the 32-row
// blocks' accumulators need the larger register budget of 6-wave workgroups)
template <int BITS, int MT>
static int launch_band_mt(const BandArgs &a, int nw, int tiles, int ksplit, hipStream_t stream) {
    if constexpr (MT <= 2) {
        if (nw == 8) return launch_band_t<BITS, MT, 8>(a, tiles, ksplit, stream);
    }
    return launch_band_t<BITS, MT, 4>(a, tiles, ksplit, stream);
}

// LDS bytes of a variant (Geo<>::LDS)
static int band_lds(int bits, int mt, int nw) {
    return band_nx(bits, mt, nw) * mt * 4096 + 3 * (32 * nw * 128) + 2 * (1024 * nw);
}

// Returns SC_EUNSUPPORTED when the shape does not suit this kernel (the caller falls
// back).  force_nw / force_split (0 = automatic) pin the plan for measurements.
// no_alloc: the split-K partials go to the allocation-free scratch array (shapes that
// need more are SC_EUNSUPPORTED) instead of the library-owned buffer.
// swiglu_half > 0: the weight is gate|up stacked (N = 2 swiglu_half) and y
// [M, swiglu_half] receives silu(gate) * up, applied by the split-K pass.
// keep (plain products): the partials are left to the caller's pass (keep->splits > 0)
// instead of being summed into y.
int launch_qgemm_band(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                      const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits, hipStream_t stream,
                      bool no_alloc, int swiglu_half, int force_nw, int force_split, SplitKeep *keep) {
    if (M < 1 || M > 256 || N < 1) return SC_EUNSUPPORTED;
    if (bits != 4 && bits != 8) return SC_EUNSUPPORTED;
    if (K % 512) return SC_EUNSUPPORTED;                 // whole 8-group scale/bias blocks
    if (swiglu_half && N != 2 * swiglu_half) return SC_EUNSUPPORTED;
    if (((uintptr_t)x % 16) || ((uintptr_t)wq % 16) || ((uintptr_t)s % 16) || ((uintptr_t)b % 16))
        return SC_EUNSUPPORTED;
    // per-lane DMA offsets are 32-bit: x rows (M K 2 bytes) and a tile's weight rows
    if ((long long)M * K * 2 >= (1LL << 31) || (long long)K >= (1LL << 23)) return SC_EUNSUPPORTED;
    const int mt = M <= 32 ? 1 : M <= 64 ? 2 : M <= 128 ? 4 : 8;
    const int G = K / 64, nb = G / 8;
    const DeviceInfo &di = device_info();
    const int P = di.num_cus;

    // Plan: 8-wave workgroups (256 rows) unless too few tiles would be left to fill the
    // CUs even with every scale/bias block a split of its own (twice over above 32 rows,
    // three quarters over up to 32: measured on the decode shapes); then the K splits
    // that bring the workgroups to about one round (two per CU for the small 4-wave
    // ones).
    int nw = force_nw ? force_nw : 8;
    if (nw != 4 && nw != 8) return set_error(SC_EINVAL, "qgemm_band: waves %d (4 or 8)", nw);
    if (!force_nw && (long)((N + 255) / 256) * nb < (mt == 1 ? 3L * P / 4 : 2L * P)) nw = 4;
    if (mt > 2) nw = 4;
    const int tiles = (N + 32 * nw - 1) / (32 * nw);
    const int per_cu = band_lds(bits, mt, nw) <= 80 * 1024 ? 2 : 1;
    int ksplit = force_split ? force_split : (int)((P * per_cu + tiles / 2) / tiles);
    if (ksplit < 1) ksplit = 1;
    if (ksplit > nb) ksplit = nb;
    const int bps = (nb + ksplit - 1) / ksplit;          // blocks per split
    ksplit = (nb + bps - 1) / bps;

    BandArgs a;
    a.x = x; a.wq = reinterpret_cast<const uint8_t *>(wq); a.s = s; a.b = b; a.bias = bias; a.y = y;
    a.partials = nullptr;
    a.M = M; a.N = N; a.K = K; a.G = G; a.gps = 8 * bps;
    const bool with_partials = ksplit > 1 || swiglu_half > 0;
    if (with_partials) {
        const size_t need = (size_t)ksplit * M * N;
        if (no_alloc) {
            if (need * sizeof(float) > (size_t)SC_QMM_NOALLOC_SCRATCH_BYTES) return SC_EUNSUPPORTED;
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
    if (bits == 4) {
        rc = mt == 1 ? launch_band_mt<4, 1>(a, nw, tiles, ksplit, stream)
           : mt == 2 ? launch_band_mt<4, 2>(a, nw, tiles, ksplit, stream)
           : mt == 4 ? launch_band_mt<4, 4>(a, nw, tiles, ksplit, stream)
                     : launch_band_mt<4, 8>(a, nw, tiles, ksplit, stream);
    } else {
        rc = mt == 1 ? launch_band_mt<8, 1>(a, nw, tiles, ksplit, stream)
           : mt == 2 ? launch_band_mt<8, 2>(a, nw, tiles, ksplit, stream)
           : mt == 4 ? launch_band_mt<8, 4>(a, nw, tiles, ksplit, stream)
                     : launch_band_mt<8, 8>(a, nw, tiles, ksplit, stream);
    }
    if (rc) return rc;
    if (keep) {
        keep->partials = with_partials ? a.partials : nullptr;
        keep->splits = with_partials ? ksplit : 0;
        if (with_partials && !swiglu_half) return SC_OK;
    }
    if (with_partials) return launch_qmm_finalize(a.partials, ksplit, M, N, bias, y, swiglu_half, stream);
    return SC_OK;
}

}  // namespace sc
