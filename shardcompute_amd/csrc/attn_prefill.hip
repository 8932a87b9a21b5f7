// Prefill attention: causal GQA attention of many new positions over the KV cache,
// the same contraction as attn_kernel in decode.hip (attention.py:437-466), built
// with MFMA accumulators in VGPRs (-mllvm -amdgpu-mfma-vgpr-form for this file):
// the softmax rescales the O^T accumulators in place, which in AGPRs costs a copy
// to VGPRs and back every block.
//
// KV cache layout per layer (capacity T_cap, a multiple of 32):
//   K  [B, Hkv, T_cap, D]  keys in rows     (operand A of S^T = K Q^T)
//   Vt [B, Hkv, D, T_cap]  values transposed (operand A of O^T = Vt P^T)
#include "sc_common.h"
#include "dma_util.h"

#include <float.h>
#include <math.h>
#include <type_traits>

namespace sc {

namespace {

// Causal GQA attention of many new positions (the same contraction as attn_kernel,
// attention.py:437-466), for head_dim 128: a workgroup owns 128 query columns, the
// R query heads of kv head hk at positions [PB qb, PB qb + PB) (PB = 128 / R; column
// c is position PB qb + c / R, head hk R + c % R), so each 64-key block of K and Vt
// staged in LDS serves 128 columns (attn_kernel's workgroups serve 16).  4 waves,
// wave w owns columns [32 w, 32 w + 32), on v_mfma_f32_32x32x16_bf16:
// * S^T[64 keys x 32 columns] = K Q^T: two 32-key blocks, 8 k-steps of 16 dims; the
//   column's q is operand B (registers, loaded once); operand A row i is key
//   swap23(i) (bits 2 and 3 of i exchanged), so that accumulator register r of lane
//   (column li, half lh) holds key 16 (r / 8) + 8 lh + r % 8 of the 32-key block:
//   every 8 registers are 8 consecutive keys;
// * online softmax per column over its 32 values and the partner lane li + 32, with
//   scores kept unscaled (one FMA folds the scale into the exponent); the running
//   maximum is only moved when it grew by more than 2^8 in probability, so that O
//   is rescaled in few blocks (probabilities stay below 256, exact in the ratio);
//   keys are masked only in the blocks that reach a column's last key;
// * O^T[128 dims x 32 columns] += Vt P^T in 4 k-steps of 16 keys: P^T is operand B
//   straight from the S^T registers (bf16), operand A one 16-byte read of 8
//   consecutive keys of a Vt row;
// * K and Vt blocks reach LDS by LDS-DMA, one block ahead in a 2-stage ring (64 KB,
//   so that two workgroups, 8 waves, share a CU and hide each other's waits), their
//   16-byte chunks XOR-swizzled by row so that every operand read is conflict-free;
// * cache slots past the length may hold anything, NaN included: their scores are
//   masked and, in the block that crosses the length, their V pieces are zeroed
//   before they meet the zero probabilities;
// * workgroups of later positions (more keys) are dispatched first, the first two
//   rounds in heavy/light pairs.
// The result is bf16(O / l) per column, as attn_kernel writes it (P in bf16, fp32
// sums), with the sums in another order.
constexpr int FA_COLS = 128, FA_KB = 64, FA_D = 128, FA_THREADS = 256;
constexpr int FA_KTILE = FA_KB * FA_D * 2;           // 16 KB: 64 keys x 256 B
constexpr int FA_VTILE = FA_D * FA_KB * 2;           // 16 KB: 128 dims x 128 B
constexpr int FA_STAGE = FA_KTILE + FA_VTILE;
constexpr int FA_NST = 2;                            // LDS stages: block blk being read, blk + 1 landing
constexpr int FA_LDS = FA_NST * FA_STAGE;            // 64 KB
constexpr int FA_SAHEAD = 4;                         // operand reads in flight ahead of the MFMAs

struct FaArgs {
    const uint16_t *q;
    long q_stride;
    const uint16_t *kc;       // [B, Hkv, T_cap, 128]
    const uint16_t *vt;       // [B, Hkv, 128, T_cap]
    const int32_t *cache_len;
    uint16_t *out;
    long out_stride;
    int S, H, Hkv, R, T_cap, nqb;
    int pair_half;            // > 0: the first 2 pair_half workgroups are dispatched in heavy/light pairs
    float scale_log2;
    // the additive mask (attn_prefill_kernel<true>): element (b, h, s, t) at
    // mask + b msb + h msh + s mss + t mst, added to the scaled scores
    const float *mask;
    long msb, msh, mss, mst;
    float mask_unscale;       // 1 / scale: a mask value in the kernel's unscaled score units
};

// exchange bits 2 and 3
__device__ __forceinline__ int fa_swap23(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }
// byte offset of 16-byte chunk c of K tile row r (16 chunks a row): chunk c of key row
// r sits at position c ^ swap23(r) % 16, so the rows swap23(i), i = 0..15, that lanes
// 0..15 of an operand read cover meet in distinct positions
__device__ __forceinline__ uint32_t fa_kswz(int r, int c) {
    return (uint32_t)(r * 256 + ((c ^ (fa_swap23(r) & 15)) << 4));
}
// byte offset of 16-byte chunk c (8 keys) of Vt tile row d (8 chunks a row),
// XOR-swizzled by d / 2 % 8.  A 16-byte read is served 16 lanes (256 bytes, every
// bank once) at a time: rows d and d + 1 lie in different halves of the banks, so
// the 16 rows of such a group meet in distinct bank groups (swizzling by d % 8 puts
// rows d and d + 8 on the same banks: 4 conflict cycles a read, measured)
__device__ __forceinline__ uint32_t fa_vswz(int d, int c) { return (uint32_t)(d * 128 + ((c ^ ((d >> 1) & 7)) << 4)); }

// ADD: the additive mask (attention.py:449-450).  Every block adds the column's mask
// row (finite values clamped to -FLT_MAX in the kernel's units, -inf kept), loaded one
// block ahead into registers; a column's running maximum may then stay -inf for whole
// blocks, so probabilities of -inf scores are set to 0 explicitly, and a column whose
// every visible score is -inf ends as 0 / 0 = NaN, as the reference's softmax does.
template <bool ADD>
__global__ void __launch_bounds__(FA_THREADS) attn_prefill_kernel(FaArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    // work rank of this workgroup (0: most keys): later positions first, over every
    // (sequence, kv head).  Two workgroups share a CU; the first 2 pair_half (two
    // per CU) are resident together, workgroup p beside p + pair_half in dispatch
    // order, so that round pairs rank j with rank 2 pair_half - 1 - j and each CU
    // gets about the same number of key blocks (a heuristic on dispatch order: any
    // order gives the same results)
    int rank = (int)blockIdx.x;
    if (a.pair_half > 0 && rank < 2 * a.pair_half && rank >= a.pair_half) rank = 3 * a.pair_half - 1 - rank;
    const int nbh = (int)(gridDim.x / a.nqb);             // B * Hkv
    const int qb = a.nqb - 1 - rank / nbh;
    const int hk = rank % nbh % a.Hkv;
    const int b = rank % nbh / a.Hkv;
    const int T = a.cache_len[0] + a.S;               // cached positions, the S new ones included
    const int off = T - a.S;
    const int PB = FA_COLS / a.R;

    const int col = 32 * w + li;
    const int pos = qb * PB + col / a.R;
    const int h = hk * a.R + col % a.R;
    const bool col_ok = pos < a.S;
    const int last_pos = min(a.S - 1, qb * PB + PB - 1);
    // last key this column sees; columns past the S positions (never written) see as
    // many as the workgroup's last position, so that every column's scores are finite
    const int limit = off + min(pos, last_pos);
    // the fewest keys a column of this wave sees (its first column's): blocks wholly
    // at or below need no mask
    const int wlimit = off + min(qb * PB + 32 * w / a.R, last_pos);

    bf16x8_t qv[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (col_ok)
            v = *reinterpret_cast<const uint4 *>(a.q + ((size_t)b * a.S + pos) * a.q_stride + (size_t)h * FA_D + 16 * ks + 8 * lh);
        qv[ks] = as_bf16x8(v);
    }
    const int kend = off + last_pos + 1;               // keys [0, kend) are needed
    const int nblk = (kend + FA_KB - 1) / FA_KB;
    const int nfull = min(nblk, (wlimit + 1) / FA_KB);  // blocks with every key <= wlimit
    const uint16_t *kbase = a.kc + ((size_t)b * a.Hkv + hk) * (size_t)a.T_cap * FA_D;
    const uint16_t *vbase = a.vt + ((size_t)b * a.Hkv + hk) * (size_t)FA_D * a.T_cap;

    // staging of a block, all by LDS-DMA (no registers; explicit vmcnt waits, the
    // only vector-memory operations of the loop): wave w issues K instructions
    // 4 w .. 4 w + 3 (4 rows each: lane i lands at row 4 q + i / 16, position i % 16)
    // and Vt instructions 4 w .. 4 w + 3 (8 rows each: lane i at row 8 q + i / 8,
    // position i % 8), each lane loading the chunk the swizzle puts at its position.
    // Blocks are issued one ahead into a 2-stage ring.
    auto stage_blk = [&](int kb, int st) {
        const uint32_t kl = (uint32_t)(uintptr_t)(smem + st * FA_STAGE);
        const uint32_t vl = kl + FA_KTILE;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int qi = 4 * w + qq;
            const int r = 4 * qi + (lane >> 4);
            const int c = (lane & 15) ^ (fa_swap23(r) & 15);
            const int key = min(kb + r, a.T_cap - 1);
            dma::dma16s(kbase, (uint32_t)(key * (FA_D * 2) + 16 * c), kl + 1024 * qi);
        }
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int qi = 4 * w + qq;
            const int d = 8 * qi + (lane >> 3);
            const int c = (lane & 7) ^ ((d >> 1) & 7);
            // T_cap is a multiple of 32, so only chunks wholly past the capacity clamp
            const int k0 = min(kb + 8 * c, a.T_cap - 8);
            dma::dma16s(vbase, (uint32_t)((d * a.T_cap + k0) * 2), vl + 1024 * qi);
        }
    };

    f32x16_t o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x16_t{};
    float m = -INFINITY, lsum = 0.f;

    // the column's mask row and the 32 values of the next block (register r of half kh:
    // key kb + 32 kh + 16 (r / 8) + 8 lh + r % 8; keys past the column's limit read the
    // limit's value, which the causal mask then replaces)
    const float *mrow = nullptr;
    float mnext[2][16];
    auto load_mask = [&](int kb) __attribute__((always_inline)) {
        if constexpr (ADD) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int t = min(kb + 32 * kh + 16 * (r >> 3) + 8 * lh + (r & 7), limit);
                    mnext[kh][r] = mrow[(long)t * a.mst];
                }
        }
    };
    if constexpr (ADD) {
        mrow = a.mask + (long)b * a.msb + (long)h * a.msh + (long)min(pos, last_pos) * a.mss;
        load_mask(0);
    }

    stage_blk(0, 0);
    // q's loads must be retired here, before the loop: the compiler cannot see the
    // DMA, and a wait it placed at q's first use would sit in the loop and also wait
    // for the blocks in flight every iteration
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) asm volatile("" ::"v"(qv[ks]));
    dma::wait_vm<0>();
    __syncthreads();
    const float sc = a.scale_log2;
    const int arow = fa_swap23(li);                    // key row of operand A in each 32-key half
    // the stage is a compile-time constant in each copy of the body, so that every
    // operand read is a loop-invariant lane offset plus an immediate
    auto block = [&](int blk, auto mask_tag, auto stage_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr int st = decltype(stage_tag)::value;
        const int kb = blk * FA_KB;
        const uint8_t *K = smem + st * FA_STAGE;
        const uint8_t *V = K + FA_KTILE;
        // block blk + 1 goes to the stage block blk - 1 used (read before the last barrier)
        if (blk + 1 < nblk) stage_blk(kb + FA_KB, st ^ 1);

        // S^T for the block's two 32-key halves: register r of sacc[kh] is key
        // kb + 32 kh + 16 (r / 8) + 8 lh + r % 8
        // (the two halves' chains interleaved, so consecutive MFMAs are independent;
        // operand reads run FA_SAHEAD ahead of their MFMAs: the scheduler, left alone,
        // issues each read just before its MFMA and waits out the LDS latency 16 times)
        f32x16_t sacc[2] = {f32x16_t{}, f32x16_t{}};
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const bf16x8_t ka = as_bf16x8(*reinterpret_cast<const uint4 *>(K + fa_kswz(32 * kh + arow, 2 * ks + lh)));
                sacc[kh] = mfma32x32x16(ka, qv[ks], sacc[kh]);
            }
#pragma unroll
        for (int i = 0; i < FA_SAHEAD; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 16 - FA_SAHEAD; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < FA_SAHEAD; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (ADD) {
            // this block's mask (landed with the previous block's closing wait), then the
            // next block's loads, which this block's closing wait retires
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float mv = mnext[kh][r];
                    sacc[kh][r] += mv == -INFINITY ? -INFINITY : fmaxf(mv * a.mask_unscale, -FLT_MAX);
                }
            if (blk + 1 < nblk) load_mask(kb + FA_KB);
        }
        if (MASK) {
            const int rel = limit - kb - 8 * lh;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (32 * kh + 16 * (r >> 3) + (r & 7) > rel) sacc[kh][r] = -INFINITY;
        }
        // the column's block maximum (this lane and li + 32), unscaled; block 0 holds
        // key 0, which every column sees, so the running maximum is finite from there on
        float bm = -INFINITY;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int r = 0; r < 16; ++r) bm = fmaxf(bm, sacc[kh][r]);
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        float alpha = 1.f;
        if ((bm - m) * sc > 8.f) {
            alpha = __builtin_amdgcn_exp2f((m - bm) * sc);
            m = bm;
        }
        const float nms = -m * sc;
        float ps = 0.f;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float p;
                if constexpr (ADD) {
                    // (score - m) sc: a column whose visible scores all sit at the clamp
                    // (-FLT_MAX) gets exp2(0) for each, uniform weights; the fused form's
                    // rounded -m sc would leave a remainder of ~1e30 there.  -inf scores
                    // get 0 (with m = -inf, -inf - m is NaN).
                    p = sacc[kh][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((sacc[kh][r] - m) * sc);
                } else {
                    p = __builtin_amdgcn_exp2f(fmaf(sacc[kh][r], sc, nms));
                }
                sacc[kh][r] = p;
                ps += p;
            }
        lsum = lsum * alpha + ps;
        // rescale O^T only when some column's maximum moved (wave-uniform test)
        if (__ballot(alpha != 1.f) != 0ull) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
        }
        // O^T += Vt P^T over 4 steps of 16 keys: step s4 takes registers 8 (s4 % 2) ..
        // + 7 of half s4 / 2, keys kb + 8 c .. + 7 with c = 4 (s4 / 2) + 2 (s4 % 2) + lh
        // (operand reads FA_SAHEAD ahead of their MFMAs, as for S^T)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int kh = s4 >> 1, r0 = 8 * (s4 & 1);
            const bf16x8_t pb = as_bf16x8(cvt_pk_bf16(sacc[kh][r0], sacc[kh][r0 + 1]),
                                          cvt_pk_bf16(sacc[kh][r0 + 2], sacc[kh][r0 + 3]),
                                          cvt_pk_bf16(sacc[kh][r0 + 4], sacc[kh][r0 + 5]),
                                          cvt_pk_bf16(sacc[kh][r0 + 6], sacc[kh][r0 + 7]));
            const int c = 4 * kh + 2 * (s4 & 1) + lh;
            // cache slots at or past T may hold anything, NaN included: their zero
            // probabilities must not meet them, so the V pieces of the block that
            // crosses T (a masked block: its keys pass every column's limit) are masked
            uint4 mk = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
            if (MASK && kb + FA_KB > T) {
                const int k0 = kb + 8 * c;
                mk.x = (k0 + 0 < T ? 0xFFFFu : 0u) | (k0 + 1 < T ? 0xFFFF0000u : 0u);
                mk.y = (k0 + 2 < T ? 0xFFFFu : 0u) | (k0 + 3 < T ? 0xFFFF0000u : 0u);
                mk.z = (k0 + 4 < T ? 0xFFFFu : 0u) | (k0 + 5 < T ? 0xFFFF0000u : 0u);
                mk.w = (k0 + 6 < T ? 0xFFFFu : 0u) | (k0 + 7 < T ? 0xFFFF0000u : 0u);
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const uint4 v = *reinterpret_cast<const uint4 *>(V + fa_vswz(32 * db + li, c));
                o[db] = mfma32x32x16(as_bf16x8(v.x & mk.x, v.y & mk.y, v.z & mk.z, v.w & mk.w), pb, o[db]);
            }
        }
#pragma unroll
        for (int i = 0; i < FA_SAHEAD; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 16 - FA_SAHEAD; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < FA_SAHEAD; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        // block blk + 1 must have landed before the barrier
        dma::wait_vm<0>();
        __syncthreads();
    };
    // the blocks below every column's limit of this wave, then those that need the mask
    // (each wave runs nblk blocks, one barrier each); block blk is in stage blk % 2
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    int blk = 0;
    for (; blk + 1 < nfull; blk += 2) {
        block(blk, std::false_type{}, S0{});
        block(blk + 1, std::false_type{}, S1{});
    }
    if (blk < nfull) block(blk++, std::false_type{}, S0{});
    for (; blk < nblk; ++blk) {
        if (blk & 1) block(blk, std::true_type{}, S1{});
        else block(blk, std::true_type{}, S0{});
    }
    const float ltot = lsum + __shfl_xor(lsum, 32);
    if (!col_ok) return;
    const float inv = (ADD || ltot > 0.f) ? 1.f / ltot : 0.f;
    uint16_t *orow = a.out + ((size_t)b * a.S + pos) * a.out_stride + (size_t)h * FA_D;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int d = 32 * db + 8 * r4 + 4 * lh;
            *reinterpret_cast<uint2 *>(orow + d) =
                make_uint2(cvt_pk_bf16(o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv),
                           cvt_pk_bf16(o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv));
        }
}

}  // namespace

// Launches attn_prefill_kernel when the shape suits it (head_dim 128, the GQA ratio
// dividing 128, 16-byte aligned Vt, at least 128 / R new positions: one workgroup's
// columns) and returns SC_OK; returns 1, launching nothing, when it does not.  The
// choice does not depend on the batch size, so that a sequence's result is the same
// alone and in a batch (every column's arithmetic is its own).  The caller has
// checked the shape, strides and pointers as launch_attention does.  mask / ms: the
// additive mask and its strides (b, h, s, t), or null.
int launch_attn_prefill(const uint16_t *q, long q_stride, const uint16_t *kc, const uint16_t *vt, long T_cap,
                        const int32_t *cache_len, uint16_t *out, long out_stride, long B, long S, long H, long Hkv,
                        long D, float scale, hipStream_t stream, const float *mask, const long *ms) {
    const long R = H / Hkv;
    if (D != FA_D || FA_COLS % R != 0 || ((uintptr_t)vt % 16) != 0) return 1;
    if (T_cap > (1L << 22)) return 1;    // staging offsets within one (b, kv head) slab are 32-bit
    const long nqb = (S + FA_COLS / R - 1) / (FA_COLS / R);
    const long wgs = B * Hkv * nqb;
    if (S < FA_COLS / R || wgs >= (1L << 31)) return 1;
    FaArgs f;
    f.q = q; f.q_stride = q_stride; f.kc = kc; f.vt = vt; f.cache_len = cache_len;
    f.out = out; f.out_stride = out_stride;
    f.S = (int)S; f.H = (int)H; f.Hkv = (int)Hkv; f.R = (int)R; f.T_cap = (int)T_cap; f.nqb = (int)nqb;
    const long per_round = 2L * device_info().num_cus;     // two workgroups per CU (64 KB LDS each)
    f.pair_half = wgs >= per_round ? (int)(per_round / 2) : 0;
    f.scale_log2 = scale * 1.4426950408889634f;
    f.mask = mask;
    f.msb = mask ? ms[0] : 0; f.msh = mask ? ms[1] : 0; f.mss = mask ? ms[2] : 0; f.mst = mask ? ms[3] : 0;
    f.mask_unscale = 1.f / scale;
    static bool configured[2] = {false, false};
    if (!configured[mask != nullptr]) {
        SC_HIP_CHECK(hipFuncSetAttribute(mask ? reinterpret_cast<const void *>(attn_prefill_kernel<true>)
                                              : reinterpret_cast<const void *>(attn_prefill_kernel<false>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, FA_LDS));
        configured[mask != nullptr] = true;
    }
    if (mask) hipLaunchKernelGGL(attn_prefill_kernel<true>, dim3((unsigned)wgs), dim3(FA_THREADS), FA_LDS, stream, f);
    else hipLaunchKernelGGL(attn_prefill_kernel<false>, dim3((unsigned)wgs), dim3(FA_THREADS), FA_LDS, stream, f);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // namespace sc
