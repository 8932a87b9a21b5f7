// The whole transformer trunk of one batch-1 decode step in one persistent launch.
//
// One step of ParallelTransformer.forward at one token (parallel/transformer.py:516-559:
// embedding, then per layer RMSNorm -> q|k|v -> RoPE + KV append + attention ->
// o_proj (+ residual) -> RMSNorm -> gate|up -> SiLU gate -> down_proj (+ residual)),
// with every projection a W4/W8 g64 mx.quantized_matmul (quantized_linear.py:168-176).
//
// Why one launch: at batch 1 every projection is a short weight stream (9-66 MB), and
// as separate launches each pays a launch boundary, a ramp and a tail in which HBM
// idles.  Here each workgroup (one per CU) streams its share of every op's weights
// (and of the attention's cached keys and values) through per-wave LDS rings without
// waiting for the data the op consumes; only the arithmetic waits.  A CU's weight
// stream for the coming ops keeps running while the step's critical path (norm ->
// products -> attention -> ...) moves from op to op.
//
// Roles inside a workgroup: 8 worker waves claim 4 KB items (16 weight rows x 256 B
// plus scales/biases, or 8 cached keys with their values) from one counter spanning
// all ops of the step, DMA them into their ring and compute them; one control wave
// polls each op's input and publishes each op's output.  While the workers compute
// an op's items the control wave publishes each projection tile as soon as its K
// chunks are counted, computes the attention items' merge weights once they are in,
// and (9 items for 8 workers) computes a unit's last attention item itself.  At each
// op boundary all nine waves meet (LDS barriers only) and share the staging work
// (norm, operand permutation, merging the workers' attention states).
//
// Workgroups exchange activations through "LL" words: 8-byte (data, epoch)
// pairs written with one agent-coherent store, so a reader that sees the epoch of
// the current op and launch also sees the data (no flags, no fences, no grid
// barrier).  Each op kind has its own exchange buffer; a buffer is rewritten one
// layer later, after every reader has passed an op that needs all workgroups'
// outputs, so no reader can see a newer write.  Every op's input is the previous
// op's output.  Epochs are unique per (launch, op).
//
// Arithmetic: the projections use the item format, MFMA math and chunk-order
// partial sums of qgemv_m1_kernel, the norm the 256-thread partition of
// add_rms_norm_kernel and the rotation rope_append_kernel's, so those results are
// bit-identical to the per-op path.  Attention (fp32 scores, softmax and
// probabilities times bf16 values) differs from attn_decode_kernel in rounding only.
//
// Every wait is bounded: on a timeout a workgroup sets the status word, skips the
// remaining work (its waves still pass every op boundary together), drains its DMA
// and ends.
#include <algorithm>
#include <cstdlib>
#include <memory>
#include <vector>

#include <type_traits>

#include "dma_util.h"
#include "../../include/shardcompute_hip.h"

namespace sc {

namespace step {

using namespace dma;

// rows of the stacked q|k|v projection
constexpr int qkv_rows(int H, int Hkv, int D) { return (H + 2 * Hkv) * D; }

constexpr int WORKERS = 8;
constexpr int CTL = WORKERS;                // the control wave
constexpr int THREADS = 64 * (WORKERS + 1);
constexpr int SLOT = 4096 + 512;            // item bytes + 16 rows x 8 groups of scales and biases
#ifndef SC_TRUNK_RING
#define SC_TRUNK_RING 3
#endif
constexpr int TRING = SC_TRUNK_RING;        // ring slots per worker wave (TRING - 1 items in flight)
constexpr unsigned long long TIMEOUT_TICKS = 20000000ull;   // 200 ms of the 100 MHz real-time clock
// head_dim D (64 or 128) and the most query heads per kv head RMAX (4 or 8) are
// template parameters of the kernel: (128, 4) for the Llama-3 shapes, (64, 8) for
// TinyLlama's

// Projection tiles per workgroup and op whose outputs the control wave publishes as
// they complete (ops with more publish at the op boundary)
constexpr int MAX_TILES = 64;
constexpr int NT = 6;                       // ops per layer, in this order:
enum OpKind { K_QKV = 0, K_ATTN = 1, K_MERGE = 2, K_O = 3, K_GU = 4, K_DOWN = 5 };
enum OpFlags { F_NORM = 1, F_SWIGLU = 2, F_RESID = 4, F_ROW8 = 8 };
enum Buf { B_H = 0, B_QKV, B_PART, B_ATT, B_HMID, B_ACT, B_COUNT };

// Shape of one of the four projections of a layer (the same in every layer).
struct GemvDesc {
    int N, K, G, T, cpt;
    unsigned cpt_magic;     // ceil(2^32 / cpt): item / cpt == umulhi(item, cpt_magic)
    int half;               // F_SWIGLU: output width (gate rows)
    int flags, in_buf, out_buf;
    const uint2 *in;        // LL words of the input and the output (exchange buffers in_buf, out_buf)
    uint2 *out;
    int rb, re, ntl;        // this workgroup's rows [rb, re), in ntl 16-row tiles from rb (set in LDS at launch)
};

// Device pointers of one layer: projections q|k|v, o, gate|up, down; norms; cache.
struct LayerPtrs {
    const uint32_t *wq[4];
    const uint16_t *s[4];
    const uint16_t *b[4];
    const uint16_t *ln[2];  // input_layernorm, post_attention_layernorm
    uint16_t *kc, *vt;      // [Hkv, T_cap, D], [Hkv, D, T_cap]
};

struct Args {
    const LayerPtrs *layers;  // [L]
    GemvDesc gd[4];           // q|k|v, o, gate|up, down
    uint2 *buf[B_COUNT];
    const int32_t *counters;  // [0]: cached positions before this token (its slot)
    uint32_t *epoch_base;     // incremented by workgroup 0 at its end
    unsigned *status;         // 0 ok; nonzero: a launch gave up
    const int32_t *ids;       // the step's token id
    const uint16_t *embed;    // [V_local, hidden]
    const float *cos_t, *sin_t;
    uint16_t *h_out;          // the last layer's output (plain bf16)
    long vocab_start;
    int V_local, table_len, pos_offset;
    int L, nops, hidden, H, Hkv, R, NR, T_cap, C_merge;
    float eps, scale_log2;
    // LDS layout (byte offsets into dynamic shared memory)
    int o_xl, o_xzero, o_xs, o_part, o_hbuf, o_qkv, o_gd, o_lp, lds_bytes;
    int o_spare;            // the control wave's attention item area (in x's), or -1
    int single_max;         // contexts up to this length use one key range per kv head
    uint32_t *trace;          // null, or [P][nops][4] real-time stamps of the last launch
};

// The exchange words are accessed through global-address-space pointers: the kernel
// reads its buffer pointers from LDS, so the compiler cannot infer the address space
// and would emit FLAT instructions, which also count against lgkmcnt.  Every LDS or
// scalar-load wait of the control wave would then wait for its outstanding exchange
// stores and polls as well.  Global instructions count against vmcnt only.
typedef __attribute__((address_space(1))) unsigned long long global_u64;

__device__ __forceinline__ void ll_store(uint2 *p, uint32_t data, uint32_t ep) {
    const unsigned long long v = (unsigned long long)data | ((unsigned long long)ep << 32);
    __hip_atomic_store((global_u64 *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long ll_load(const uint2 *p) {
    return __hip_atomic_load((const global_u64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long now() { return __builtin_amdgcn_s_memrealtime(); }

// Tiles [tb, te) of a projection with T tiles owned by workgroup wg of P.
__device__ __forceinline__ void gemv_tiles(int T, int wg, int P, int &tb, int &te) {
    tb = (int)((unsigned)wg * (unsigned)T / (unsigned)P);
    te = (int)((unsigned)(wg + 1) * (unsigned)T / (unsigned)P);
}

// Rows [rb, re) of a projection owned by workgroup wg of P, covered by ntl 16-row
// tiles from rb: contiguous ranges of whole tiles, or with F_ROW8 of 8-row halves,
// when that evens out the rows per workgroup (q|k|v's 384 tiles on 256 CUs: 24 rows
// each instead of 16 or 32).  A last tile with 8 rows loads its last row in place of
// the 8 it does not own and publishes only its own rows.  SwiGLU tiles (8 gate + 8 up
// rows) are whole tiles, with rb = 16 x the first tile.
__device__ __forceinline__ void gemv_rows(const GemvDesc &g, int wg, int P, int &rb, int &re, int &ntl) {
    int b, e;
    if (g.flags & F_ROW8) {
        gemv_tiles((g.N + 7) >> 3, wg, P, b, e);
        rb = 8 * b;
        re = min(8 * e, g.N);
        ntl = (e - b + 1) >> 1;
    } else {
        gemv_tiles(g.T, wg, P, b, e);
        rb = 16 * b;
        re = min(16 * e, g.N);
        ntl = e - b;
    }
}

__device__ __forceinline__ int gemv_index(int kind) {
    return kind == K_QKV ? 0 : kind == K_O ? 1 : kind == K_GU ? 2 : 3;
}

// v equal within each group of 8 lanes: sum / max over the 8 groups
__device__ __forceinline__ float groups_sum(float v) {
    float a, b;
    v += dpp_mov<DPP_ROR8>(v);
    swap16(v, a, b);
    swap32(a + b, a, b);
    return a + b;
}
__device__ __forceinline__ float groups_max(float v) {
    float a, b;
    v = fmaxf(v, dpp_mov<DPP_ROR8>(v));
    swap16(v, a, b);
    swap32(fmaxf(a, b), a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float lanes_sum(float v) { return groups_sum(group8_sum(v)); }
__device__ __forceinline__ float lanes_max(float v) {
    v = fmaxf(v, dpp_mov<DPP_XOR1>(v));
    v = fmaxf(v, dpp_mov<DPP_XOR2>(v));
    return groups_max(fmaxf(v, dpp_mov<DPP_HALF_MIRROR>(v)));
}

// Columns (p[16 ch], p[16 ch + 1]) summed over the tile's K chunks ch < cpt in chunk
// order (qgemv_m1_kernel's order, so the bits match), the LDS reads issued 8 chunks
// at a time.
__device__ __forceinline__ void chunk_sums(const float *p, int cpt, float &s0, float &s1) {
    int ch = 0;
    for (; ch + 8 <= cpt; ch += 8) {
        float2 t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = *reinterpret_cast<const float2 *>(p + (ch + k) * 16);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            s0 += t[k].x;
            s1 += t[k].y;
        }
    }
    for (; ch < cpt; ++ch) {
        const float2 t = *reinterpret_cast<const float2 *>(p + ch * 16);
        s0 += t.x;
        s1 += t.y;
    }
}

struct AttnUnit {
    int valid, kvh, r, lo, hi;   // keys [lo, hi) of kv head kvh (hi includes the new position)
};

__device__ __forceinline__ AttnUnit attn_unit(const Args &a, int wg, int T, int kps) {
    AttnUnit u;
    u.valid = wg < a.Hkv * a.NR;
    u.kvh = u.valid ? wg / a.NR : 0;
    u.r = u.valid ? wg - u.kvh * a.NR : 0;
    u.lo = u.r * kps;
    u.hi = min(u.lo + kps, T);
    return u;
}

}  // namespace step

using namespace step;

template <int BITS, int D, int RMAX>
__global__ void __launch_bounds__(THREADS) decode_step_kernel(Args a) {
    static_assert(D == 64 || D == 128, "head_dim");
    static_assert(RMAX <= 16, "query heads per kv head (one MFMA tile of columns)");
    constexpr int SPAN_K = BITS == 4 ? 128 : 64;
    constexpr int SPAN_GROUPS = SPAN_K / 64;
    constexpr int SPAN_WORDS = SPAN_K / 8;
    constexpr int ITEM_K = 4 * SPAN_K;
    constexpr int ITEM_GROUPS = ITEM_K / 64;
    constexpr int MFMAS = BITS == 4 ? 4 : 2;
    constexpr int KCH = D / 8;              // 16-byte chunks of a key row
    constexpr int AST = RMAX * (D + 4);     // floats per attention item state: [RMAX][D + 4] = O, m, l, pad

    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ctr;                   // next stream item to claim
    __shared__ int s_pre[NT + 1];           // this workgroup's items per layer, prefix over op kinds
    __shared__ int s_total;
    __shared__ int s_abort;                 // a poll gave up: every wave skips the remaining work
    __shared__ int s_tile[MAX_TILES];       // per projection tile of the current op: chunks computed
    __shared__ float s_red[NORM_THREADS / 64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int P = gridDim.x, wg = blockIdx.x;
    const int nops = a.nops;

    uint4 *xl = reinterpret_cast<uint4 *>(smem + a.o_xl);
    uint4 *xzero = reinterpret_cast<uint4 *>(smem + a.o_xzero);
    float *xs = reinterpret_cast<float *>(smem + a.o_xs);
    float *part = reinterpret_cast<float *>(smem + a.o_part);
    uint4 *hbuf = reinterpret_cast<uint4 *>(smem + a.o_hbuf);
    uint16_t *qkv_l = reinterpret_cast<uint16_t *>(smem + a.o_qkv);   // q [RMAX][D], k [D], v [D] (bf16)
    GemvDesc *sgd = reinterpret_cast<GemvDesc *>(smem + a.o_gd);
    LayerPtrs *slp = reinterpret_cast<LayerPtrs *>(smem + a.o_lp);
    float *ast = reinterpret_cast<float *>(smem + a.o_xl);              // attention states (overlay x)

    const int pos = a.counters[0];
    const int T = pos + 1;                  // keys after the append
    // Keys per attention unit: the context split over NR ranges per kv head, or, for
    // contexts up to single_max, one range holding every key: its unit then finishes
    // the attention itself and the merge op has nothing to do (its exchange and
    // boundary cost more than a second round of items).
    // (compiled for head_dim 64 only: in the 128 instantiation the extra code cost the
    // Llama-3-8B step 0.8 %, and its contexts above 2048 positions never use it)
    const bool single = D == 64 && T <= a.single_max;
    int kps = single ? T : (T + a.NR - 1) / a.NR;
    kps = (kps + 7) & ~7;
    const uint32_t base = a.epoch_base[0];
    const AttnUnit au = attn_unit(a, wg, T, kps);
    // The unit's attention items.  With more than there are workers (9 for 8 workers
    // at 2049-2304 positions on the Llama-3-8B shape), the control wave, idle while
    // the items are computed, takes the last one: loaded into its own LDS area while
    // q|k|v is computed, so the op needs one round of items instead of two.
    const int ni_unit = au.valid && au.hi > au.lo ? (au.hi - au.lo + 7) >> 3 : 0;
    // (head_dim 128 only: at 64, with 8 query heads per kv head, the states of 9 items
    // fill the x area of TinyLlama-sized layers, so the item area would not fit)
    const bool ctl_item = D == 128 && !single && a.o_spare >= 0 && ni_unit > WORKERS;

    // ---- set-up by the control wave: shapes and layer pointers into LDS, this
    // workgroup's items per op kind; then the one workgroup-wide barrier
    if (wave == WORKERS) {
        {
            const uint4 *src = reinterpret_cast<const uint4 *>(a.layers);
            uint4 *dst = reinterpret_cast<uint4 *>(slp);
            const int n = a.L * (int)(sizeof(LayerPtrs) / 16);
            for (int c = lane; c < n; c += 64) dst[c] = src[c];
        }
        if (lane < 4) {
            GemvDesc g = lane == 0 ? a.gd[0] : lane == 1 ? a.gd[1] : lane == 2 ? a.gd[2] : a.gd[3];
            gemv_rows(g, wg, P, g.rb, g.re, g.ntl);
            sgd[lane] = g;
        }
        if (lane == 0) {
            // a cache slot outside the cache or the rotary table (a stale replay): the
            // workers get no items (no DMA is issued) and the launch ends at once
            const bool valid = pos >= 0 && pos < a.T_cap && pos + a.pos_offset < a.table_len;
            int acc = 0;
            for (int k = 0; k < NT; ++k) {
                s_pre[k] = acc;
                int n = 0;
                if (k == K_ATTN) {
                    n = ni_unit - (ctl_item ? 1 : 0);
                } else if (k != K_MERGE) {
                    const int gi = gemv_index(k);
                    const GemvDesc g = gi == 0 ? a.gd[0] : gi == 1 ? a.gd[1] : gi == 2 ? a.gd[2] : a.gd[3];
                    int rb, re, nt;
                    gemv_rows(g, wg, P, rb, re, nt);
                    n = nt * g.cpt;
                }
                acc += n;
            }
            s_pre[NT] = acc;
            s_total = valid ? acc * a.L : 0;
            s_ctr = (TRING - 1) * WORKERS;
            s_abort = valid ? 0 : 1;
            if (!valid) __hip_atomic_store(a.status, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        for (int c = lane; c < 4 * SPAN_WORDS; c += 64) xzero[c] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();

    // ====================================================================== op boundaries
    //
    // Every wave calls boundary(jj) for jj = 0 .. nops in order, exactly once each
    // (workers as soon as their next item belongs to op jj or later, so all their
    // items of op jj - 1 are computed).  boundary(jj) finishes op jj - 1 (reduces its
    // partials and publishes its output) and stages op jj's input in LDS.  The control
    // wave publishes, polls narrow inputs and appends to the cache; every wave polls
    // wide inputs.  __syncthreads waits on LDS only.

    const unsigned long long t_start = now();
    auto timed_out = [&]() -> bool {
        if (now() - t_start > TIMEOUT_TICKS) {
            __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return true;
        }
        return false;
    };

    // Control wave: gather n8 chunks of 8 bf16 (chunk c = LL words [addr(c), +4)) that
    // carry epoch ep; put(c, v) receives each chunk once (per lane; no cross-lane
    // operations inside).  Batches of 4 chunks per lane, two batches in flight (one
    // round trip for inputs that are already published); later passes re-read the
    // batches still missing a chunk.
    auto ll_gather = [&](auto addr, int n8, uint32_t ep, auto put) __attribute__((always_inline)) -> bool {
        constexpr int CPL = 4;                           // chunks per lane per batch
        constexpr int BCH = 64 * CPL;                    // chunks per batch
        const int nb = (n8 + BCH - 1) / BCH;             // at most 8 (host: widths <= 16384)
        uint32_t pend = 0u;                              // bit CPL bi + i: chunk bi * BCH + 64 i + lane missing
        for (int bi = 0; bi < nb; ++bi)
#pragma unroll
            for (int i = 0; i < CPL; ++i)
                if (bi * BCH + i * 64 + lane < n8) pend |= 1u << (CPL * bi + i);
        auto load = [&](int bi, unsigned long long (&v)[4 * CPL]) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const uint2 *p = addr(min(bi * BCH + i * 64 + lane, n8 - 1));
#pragma unroll
                for (int k = 0; k < 4; ++k) v[4 * i + k] = ll_load(p + k);
            }
        };
        auto check = [&](int bi, const unsigned long long (&v)[4 * CPL]) __attribute__((always_inline)) {
            const uint32_t pb = (pend >> (CPL * bi)) & ((1u << CPL) - 1u);
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                if (pb & (1u << i)) {
                    bool okc = true;
#pragma unroll
                    for (int k = 0; k < 4; ++k) okc = okc && (uint32_t)(v[4 * i + k] >> 32) == ep;
                    if (okc) {
                        put(bi * BCH + i * 64 + lane, make_uint4((uint32_t)v[4 * i], (uint32_t)v[4 * i + 1],
                                                               (uint32_t)v[4 * i + 2], (uint32_t)v[4 * i + 3]));
                        pend &= ~(1u << (CPL * bi + i));
                    }
                }
            }
        };
        unsigned long long va[4 * CPL], vb[4 * CPL];
        load(0, va);
        for (int bi = 0; bi < nb; bi += 2) {
            if (bi + 1 < nb) load(bi + 1, vb);
            check(bi, va);
            if (bi + 2 < nb) load(bi + 2, va);
            if (bi + 1 < nb) check(bi + 1, vb);
        }
        // later passes: the batches still missing a chunk, two at a time (one round trip
        // per pair)
        for (int it = 0; __ballot(pend != 0u) != 0ull; ++it) {
            for (int bi = 0; bi < nb; bi += 2) {
                const bool p0 = __ballot(((pend >> (CPL * bi)) & ((1u << CPL) - 1u)) != 0u) != 0ull;
                const bool p1 =
                    bi + 1 < nb && __ballot(((pend >> (CPL * (bi + 1))) & ((1u << CPL) - 1u)) != 0u) != 0ull;
                if (p0) load(bi, va);
                if (p1) load(bi + 1, vb);
                if (p0) check(bi, va);
                if (p1) check(bi + 1, vb);
            }
            if ((it & 15) == 15 && (timed_out() ||
                __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
                return false;
        }
        return true;
    };

    // the wait limit without recording it (the workers' copy: the control wave sets the
    // status word for an aborted launch)
    auto expired = [&]() -> bool { return now() - t_start > TIMEOUT_TICKS; };

    // Every wave: gather the raw chunks of a wide input (chunk c = LL words [4c, 4c + 4) of
    // src) into x, the blocks of 64 chunks dealt round-robin to the nine waves (at most 4
    // per wave).  A chunk is watched through its last word only, with a short sleep
    // between polls, and read whole once that word carries the epoch: 2304 waves reading
    // whole inputs flood the memory path ahead of the producers' publishes and weight
    // reads.  Even a first whole read is not worth its bytes: the waves get here right
    // after their own workgroup's last item, before most producers have published
    // (8B step 1.674 -> 1.634 ms, TinyLlama 0.764 -> 0.741 ms against reading every chunk
    // whole first).  A worker's waits here also cover its older weight DMA (vmcnt retires
    // in order).
    auto gather_all = [&](const uint2 *src, int n8, uint32_t ep) __attribute__((always_inline)) -> bool {
        constexpr int NW = WORKERS + 1;
        uint32_t pend = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if ((wave + NW * i) * 64 + lane < n8) pend |= 1u << i;
        uint32_t fetch = 0u;                            // chunks to read whole this round
        const uint2 *wsrc = src + 4 * 64 * wave;        // wave-uniform base + lane offset
        const uint32_t lane_w = 4u * lane;
        for (int it = 0;; ++it) {
            unsigned long long v[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint2 *p = wsrc + 4 * 64 * NW * i + lane_w;
#pragma unroll
                for (int k = 0; k < 4; ++k) v[4 * i + k] = (fetch & (1u << i)) ? ll_load(p + k) : 0ull;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (fetch & (1u << i)) {
                    bool okc = true;
#pragma unroll
                    for (int k = 0; k < 4; ++k) okc = okc && (uint32_t)(v[4 * i + k] >> 32) == ep;
                    if (okc) {
                        xl[(wave + NW * i) * 64 + lane] = make_uint4((uint32_t)v[4 * i], (uint32_t)v[4 * i + 1],
                                                                    (uint32_t)v[4 * i + 2], (uint32_t)v[4 * i + 3]);
                        pend &= ~(1u << i);
                    }
                }
            }
            if (__ballot(pend != 0u) == 0ull) return true;
            fetch = 0u;
            for (int sp = 0;; ++sp) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (pend & (1u << i)) {
                        const uint2 *p = wsrc + 4 * 64 * NW * i + lane_w;
                        if ((uint32_t)(ll_load(p + 3) >> 32) == ep) fetch |= 1u << i;
                    }
                }
                if (__ballot(fetch != 0u) != 0ull) break;
                __builtin_amdgcn_s_sleep(2);
                if ((sp & 15) == 15 && (expired() ||
                    __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
                    return false;
            }
            if ((it & 15) == 15 && (expired() ||
                __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
                return false;
        }
    };

    // x chunk c of a projection input into LDS: W4 operand permutation + 64-element
    // group sums (the 8 chunks of a group in 8 adjacent lanes); lanes converged
    auto put_x = [&](int c, uint4 v) {
        xl[c] = BITS == 4 ? perm_w4x(v) : v;
        float g = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) g += bfe(v, e);
        g = group8_sum(g);
        if ((c & 7) == 0) xs[c >> 3] = g;
    };

    auto epoch = [&](int j) -> uint32_t { return base * (uint32_t)nops + (uint32_t)j + 1u; };
    // Op timeline (when the plan traces): per (workgroup, op) the 100 MHz real-time
    // clock when the op's items were all computed (0), its output published (1), its
    // input polled (2) and staged (3); the control wave stamps them.
    auto stamp = [&](int j, int k) __attribute__((always_inline)) {
        if (a.trace && lane == 0 && j >= 0 && j < nops)
            a.trace[((size_t)wg * nops + j) * 4 + k] = (uint32_t)__builtin_amdgcn_s_memrealtime();
    };
    auto kind_of = [&](int j) -> int { return j == 0 ? -1 : (j - 1) % NT; };

    // Control wave: publish projection op kp's tiles [t0, t1) of layer lp_ (each tile's
    // K-chunk partials summed in chunk order from part; SwiGLU, residual add and the
    // last layer's plain copy applied).
    auto publish_tiles = [&](int kp, int lp_, uint32_t ep, int t0, int t1) __attribute__((always_inline)) {
        const GemvDesc &o = sgd[gemv_index(kp)];
        const int cpt = o.cpt;
        uint2 *dst = o.out;
        uint16_t *plain = (kp == K_DOWN && lp_ == a.L - 1) ? a.h_out : nullptr;
        if (o.flags & F_SWIGLU) {
            // tile tl: gate columns 8 (tb + tl) + c, c < 8; 4 words per tile
            for (int wdx = 4 * t0 + lane; wdx < t1 * 4; wdx += 64) {
                const int tl = wdx >> 2, c = 2 * (wdx & 3);
                const float *pp = part + (size_t)tl * cpt * 16;
                float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
                chunk_sums(pp + c, cpt, g0, g1);
                chunk_sums(pp + 8 + c, cpt, u0, u1);
                const uint32_t o0 = f2bf(silu_mul_f(bf2f(f2bf(g0)), bf2f(f2bf(u0))));
                const uint32_t o1 = f2bf(silu_mul_f(bf2f(f2bf(g1)), bf2f(f2bf(u1))));
                ll_store(dst + (((o.rb >> 4) + tl) * 8 + c) / 2, o0 | (o1 << 16), ep);
            }
        } else {
            const uint32_t *hw = reinterpret_cast<const uint32_t *>(hbuf);
            const bool resid = o.flags & F_RESID;
            for (int wdx = 8 * t0 + lane; wdx < t1 * 8; wdx += 64) {
                const int tl = wdx >> 3, c = 2 * (wdx & 7);
                const int n = o.rb + tl * 16 + c;
                if (n >= o.re) continue;                    // a half tile's duplicate rows
                const float *pp = part + (size_t)tl * cpt * 16;
                float v0 = 0.f, v1 = 0.f;
                chunk_sums(pp + c, cpt, v0, v1);
                uint32_t o0 = f2bf(v0), o1 = f2bf(v1);
                if (resid) {
                    const uint32_t hv = hw[n / 2];
                    o0 = f2bf(add_rn(bf2f(hv & 0xFFFFu), bf2f(o0)));
                    o1 = f2bf(add_rn(bf2f(hv >> 16), bf2f(o1)));
                }
                ll_store(dst + n / 2, o0 | (o1 << 16), ep);
                if (plain) *reinterpret_cast<uint32_t *>(plain + n) = o0 | (o1 << 16);
            }
        }
    };
    int early_done = -1;                    // (control wave) the op whose tiles are all published

    // is_ctl: std::true_type in the control wave's copy, std::false_type in the
    // workers' (the control wave's polls then cost the workers no registers)
    auto boundary = [&](int jj, auto is_ctl) __attribute__((always_inline)) {
        constexpr bool ctl = decltype(is_ctl)::value;
        __syncthreads();                                             // B1: op jj - 1 computed
        // The control wave's publish and poll are on the step's critical path, and it
        // shares a SIMD with two workers: at the default priority their issue starves
        // it (its publish measured 2.6x slower).  It raises its priority until the
        // op's input is staged.
        if (ctl) __builtin_amdgcn_s_setprio(3);
        const int jp = jj - 1;
        if (ctl) stamp(jp, 0);
        // ------------------------------------------------------------ finish op jp
        if (jp >= 0 && !s_abort) {
            const int kp = kind_of(jp);
            const int lp_ = jp == 0 ? -1 : (jp - 1) / NT;
            const uint32_t ep = epoch(jp);
            if (kp == K_ATTN) {
                if (au.valid) {
                    // merge the items' (m, l, O) per head, in item order (the same sums
                    // whichever wave computed which item), into the unit's [R][D + 2]
                    // words: O (unnormalised), m, l.  The control wave has put each
                    // item's weight exp2(m_i - M) per head in part (fac[h][i], the head's
                    // maximum M after them) as the items completed; one fma per item and
                    // value here.
                    const int ni = ni_unit;
                    uint2 *dst = a.buf[B_PART] + (size_t)(au.kvh * a.NR + au.r) * a.R * (D + 2);
                    const float *fac = part, *mh = part + a.R * ni;
                    if (single) {
                        // the kv head's one range: the attention output itself, O / l in
                        // bf16 as the merge computes it for a single range (weight 1, the
                        // range's l), published as the merge op's output
                        if (au.r == 0) {
                            for (int t = tid; t < a.R * (D / 2); t += THREADS) {
                                const int h = t / (D / 2), x = 2 * (t - h * (D / 2));
                                const float *src = ast + h * (D + 4) + x, *fh = fac + h * ni;
                                float o0 = 0.f, o1 = 0.f, l = 0.f;
                                for (int w = 0; w < ni; ++w) {
                                    o0 = fmaf(fh[w], src[w * AST], o0);
                                    o1 = fmaf(fh[w], src[w * AST + 1], o1);
                                    l = fmaf(fh[w], src[w * AST + (D + 1 - x)], l);
                                }
                                const float inv = 1.f / l;
                                ll_store(a.buf[B_ATT] + ((size_t)(au.kvh * a.R + h) * D + x) / 2,
                                         pack_bf16x2(o0 * inv, o1 * inv), epoch(jp + 1));
                            }
                        }
                    } else
                    for (int t = tid; t < a.R * (D + 2); t += THREADS) {
                        const int h = t / (D + 2), x = t - h * (D + 2);
                        float acc = 0.f;
                        if (x == D) {
                            acc = ni > 0 ? mh[h] : -INFINITY;
                        } else {
                            const float *src = ast + h * (D + 4) + x;          // x = D + 1: l
                            const float *fh = fac + h * ni;
                            int w = 0;
                            for (; w + 4 <= ni; w += 4) {          // reads 4 items at a time
                                float f[4], o[4];
#pragma unroll
                                for (int k = 0; k < 4; ++k) {
                                    f[k] = fh[w + k];
                                    o[k] = src[(w + k) * AST];
                                }
#pragma unroll
                                for (int k = 0; k < 4; ++k) acc = fmaf(f[k], o[k], acc);
                            }
                            for (; w < ni; ++w) acc = fmaf(fh[w], src[w * AST], acc);
                        }
                        ll_store(dst + t, __float_as_uint(acc), ep);    // each thread publishes its value
                    }
                }
            } else if (kp != K_MERGE && ctl) {
                if (jp == 0) {
                    // this workgroup's words of the hidden row: masked gather (embedding.py:322-356)
                    const int words = a.hidden / 2;
                    const int per = (words + P - 1) / P;
                    const int id = a.ids[0];
                    const long local = (long)id - a.vocab_start;
                    const bool inr = local >= 0 && local < a.V_local;
                    const uint32_t *row =
                        reinterpret_cast<const uint32_t *>(a.embed + (inr ? local : 0) * (size_t)a.hidden);
                    for (int w = wg * per + lane; w < min(words, (wg + 1) * per); w += 64)
                        ll_store(a.buf[B_H] + w, inr ? row[w] : 0u, ep);
                } else if (jp != early_done) {
                    publish_tiles(kp, lp_, ep, 0, sgd[gemv_index(kp)].ntl);
                }
            }
        }
        if (ctl) stamp(jp, 1);
        if (jj >= nops) {
            if (ctl) __builtin_amdgcn_s_setprio(0);
            return;
        }
        // ------------------------------------------------------------ stage op jj
        const int k = kind_of(jj);
        const int l = jj == 0 ? -1 : (jj - 1) / NT;
        const uint32_t ep_in = epoch(jj - 1);                        // every op reads the previous op's output
        const bool is_gemv = k == K_QKV || k == K_O || k == K_GU || k == K_DOWN;
        if (ctl && (is_gemv || k == K_ATTN))
            for (int t = lane; t < MAX_TILES; t += 64) s_tile[t] = 0;   // the workers count after B3
        const GemvDesc &o = sgd[is_gemv ? gemv_index(k) : 0];
        const int W = o.K >> 3;
        const bool wide = is_gemv && !(o.flags & F_NORM) && W > 512;     // every wave polls
        if (wide && !s_abort) {
            if (!gather_all(o.in, W, ep_in) && lane == 0) s_abort = 1;
            // the workers' poll loads retire behind their weight DMA: retire them here,
            // so that no wait for them is left at the join for the other ops' paths
            wait_vm<0>();
        } else if (ctl && !s_abort) {
            bool ok = true;
            if (is_gemv) {
                const uint2 *src = o.in;
                auto addr = [&](int c) -> const uint2 * { return src + 4 * (size_t)c; };
                if (o.flags & F_NORM) {
                    // the norm weight lands in x's LDS (chunk c at x[c]) while the input is
                    // polled; the transform overwrites chunk c only after reading it
                    const uint8_t *nw = reinterpret_cast<const uint8_t *>(slp[l].ln[k == K_QKV ? 0 : 1]);
                    const uint32_t xl_lds = (uint32_t)(uintptr_t)xl;
                    for (int c0 = 0; c0 < W; c0 += 64) dma16(nw + (size_t)(c0 + lane) * 16, xl_lds + c0 * 16);
                    // raw h into hbuf (kept for the residual epilogue)
                    ok = ll_gather(addr, W, ep_in, [&](int c, uint4 v) { hbuf[c] = v; });
                    wait_vm<0>();
                } else {
                    ok = ll_gather(addr, W, ep_in, [&](int c, uint4 v) { xl[c] = v; });
                }
            } else if (k == K_ATTN) {
                if (au.valid) {
                    const int rpos = pos + a.pos_offset;
                    const float *ct = a.cos_t + (size_t)rpos * (D / 2), *st = a.sin_t + (size_t)rpos * (D / 2);
                    const int li = lane < D / 2 ? lane : 0;
                    const float cv = ct[li], sv = st[li];         // loads overlap the poll
                    const uint2 *src = a.buf[B_QKV];
                    const int qc = a.R * D / 8;                 // q chunks, then k (D / 8), then v (D / 8)
                    auto addr = [&](int c) -> const uint2 * {
                        size_t e;
                        if (c < qc) e = (size_t)(au.kvh * a.R) * D + (size_t)c * 8;
                        else if (c < qc + D / 8) e = (size_t)(a.H + au.kvh) * D + (size_t)(c - qc) * 8;
                        else e = (size_t)(a.H + a.Hkv + au.kvh) * D + (size_t)(c - qc - D / 8) * 8;
                        return src + e / 2;
                    };
                    uint4 *raw = reinterpret_cast<uint4 *>(qkv_l);
                    ok = ll_gather(addr, qc + 2 * (D / 8), ep_in, [&](int c, uint4 v) {
                        raw[c < qc ? c : RMAX * D / 8 + (c - qc)] = v;      // q heads, then k at RMAX, v after it
                    });
                    if (ok) {
                        // rotate the q heads and the new key in place (rope_append_kernel's
                        // arithmetic): lane = dim i of the first half, pairs (i, i + D/2)
                        if (lane < D / 2) {
                            for (int h = 0; h <= a.R; ++h) {
                                uint16_t *row = qkv_l + (h < a.R ? h * D : RMAX * D);
                                const float x1 = bf2f(row[lane]), x2 = bf2f(row[lane + D / 2]);
                                row[lane] = (uint16_t)f2bf(add_rn(mul_rn(x1, cv), mul_rn(-x2, sv)));
                                row[lane + D / 2] = (uint16_t)f2bf(add_rn(mul_rn(x2, cv), mul_rn(x1, sv)));
                            }
                        }
                        // the unit holding the new position appends it to the cache
                        if (au.lo <= T - 1 && T - 1 < au.hi) {
                            // global stores (the pointers come from LDS: as FLAT stores they
                            // would also hold up this wave's LDS waits until they complete,
                            // and the value column's 128 two-byte stores take long)
                            typedef __attribute__((address_space(1))) uint16_t g_u16;
                            g_u16 *kd = (g_u16 *)(slp[l].kc + ((size_t)au.kvh * a.T_cap + (T - 1)) * D);
                            g_u16 *vd = (g_u16 *)(slp[l].vt + (size_t)au.kvh * D * a.T_cap + (T - 1));
                            const uint16_t *kr = qkv_l + RMAX * D, *vr = qkv_l + RMAX * D + D;
#pragma unroll
                            for (int i = lane; i < D; i += 64) {
                                kd[i] = kr[i];
                                vd[(size_t)i * a.T_cap] = vr[i];
                            }
                        }
                    }
                }
            } else if (k == K_MERGE) {
                // attention output values [c0, c0 + C) of [H * D]: lane r < NR reads range r's
                // (m, l) and its C values of O, then the ranges merge across lanes
                const int C = a.C_merge;
                const int c0 = wg * C;
                if (!single && c0 < a.H * D) {
                    const int hq = c0 / D, d0 = c0 - hq * D;
                    const int kvh = hq / a.R, hr = hq - kvh * a.R;
                    const uint2 *src = a.buf[B_PART];
                    const bool act = lane < a.NR;
                    const size_t wb = ((size_t)(kvh * a.NR + min(lane, a.NR - 1)) * a.R + hr) * (D + 2);
                    // word pairs: pair 0 = (m, l); pair i >= 1 = O values d0 + 2 (i - 1), + 1.
                    // Values go in batches of 16 (C up to 32): the first batch is polled
                    // with (m, l), each batch is merged and published before the next is
                    // read, so only one batch is held in registers.
                    float mv = -INFINITY, lv = 0.f, ov[16];
                    // poll pairs [p0, p0 + n) (n <= 9) until every one carries the epoch
                    auto poll = [&](int p0, int n) __attribute__((always_inline)) -> bool {
                        uint32_t pend = act ? ((1u << n) - 1u) : 0u;
#pragma unroll
                        for (int d = 0; d < 16; ++d) ov[d] = 0.f;
                        for (int it = 0;; ++it) {
                            unsigned long long v[18];
#pragma unroll
                            for (int i = 0; i < 9; ++i) {
                                const int pi = p0 + i;
                                const uint2 *p = src + wb + (pi == 0 ? D : d0 + 2 * (pi - 1));
                                if (i < n) {
                                    v[2 * i] = ll_load(p);
                                    v[2 * i + 1] = ll_load(p + 1);
                                } else {
                                    v[2 * i] = v[2 * i + 1] = 0ull;
                                }
                            }
#pragma unroll
                            for (int i = 0; i < 9; ++i) {
                                if ((pend & (1u << i)) && (uint32_t)(v[2 * i] >> 32) == ep_in &&
                                    (uint32_t)(v[2 * i + 1] >> 32) == ep_in) {
                                    const float f0 = __uint_as_float((uint32_t)v[2 * i]);
                                    const float f1 = __uint_as_float((uint32_t)v[2 * i + 1]);
                                    if (p0 + i == 0) {
                                        mv = f0;
                                        lv = f1;
                                    } else {
                                        // value pair p0 + i - 1 of the batch starting at pair p0
                                        const int q = p0 == 0 ? i - 1 : i;
                                        ov[2 * q] = f0;
                                        ov[2 * q + 1] = f1;
                                    }
                                    pend &= ~(1u << i);
                                }
                            }
                            if (__ballot(pend != 0u) == 0ull) return true;
                            if ((it & 15) == 15 && (timed_out() ||
                                __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
                                return false;
                        }
                    };
                    float wr = 0.f, inv = 0.f;
                    for (int b0 = 0; ok && b0 < C; b0 += 16) {
                        const int nb = min(16, C - b0);            // values in this batch
                        ok = b0 == 0 ? poll(0, 1 + nb / 2) : poll(1 + b0 / 2, nb / 2);
                        if (!ok) break;
                        if (b0 == 0) {
                            if (!act) {
                                mv = -INFINITY;
                                lv = 0.f;
                            }
                            const float M = lanes_max(mv);
                            wr = (mv == -INFINITY) ? 0.f : exp2f(mv - M);
                            const float L = lanes_sum(act ? wr * lv : 0.f);
                            inv = 1.f / L;
                        }
                        float lo = 0.f, hi = 0.f;                // lane d / 2 keeps values b0 + d, + 1
#pragma unroll
                        for (int d = 0; d < 16; d += 2) {
                            if (d < nb) {
                                const float s0 = lanes_sum(act ? wr * ov[d] : 0.f);
                                const float s1 = lanes_sum(act ? wr * ov[d + 1] : 0.f);
                                if (2 * lane == d) {
                                    lo = s0;
                                    hi = s1;
                                }
                            }
                        }
                        if (lane < nb / 2)
                            ll_store(a.buf[B_ATT] + (c0 + b0) / 2 + lane, pack_bf16x2(lo * inv, hi * inv), epoch(jj));
                    }
                }
            }
            if (!ok && lane == 0) s_abort = 1;
        }
        if (ctl) stamp(jj, 2);
        __syncthreads();                                             // B2: raw input staged
        if (s_abort) {
            if (ctl) __builtin_amdgcn_s_setprio(0);
            __syncthreads();
            return;
        }
        if (is_gemv) {
            if (o.flags & F_NORM) {
                // RMSNorm with add_rms_norm_kernel's partition: thread t < 256 sums chunks
                // t, t + 256, ...; the 4 wave sums are added in order
                if (tid < NORM_THREADS) {
                    float ss = 0.f;
                    for (int c = tid; c < W; c += NORM_THREADS) ss = sumsq_bf16x8(ss, hbuf[c]);
                    ss = wave_sum(ss);
                    if (lane == 0) s_red[wave] = ss;
                }
                __syncthreads();
                float tot = 0.f;
#pragma unroll
                for (int i = 0; i < NORM_THREADS / 64; ++i) tot += s_red[i];
                const float root = rms_root(tot, o.K, a.eps);
                for (int c = tid; c < W; c += THREADS) put_x(c, norm_bf16x8(hbuf[c], xl[c], root));
            } else {
                for (int c = tid; c < W; c += THREADS) put_x(c, xl[c]);
            }
        }
        if (ctl) __builtin_amdgcn_s_setprio(0);
        __syncthreads();                                             // B3: op jj's input ready
        if (ctl) stamp(jj, 3);
    };

    // ====================================================================== item stream
    // Stream item g of this workgroup -> (layer l, op kind k, item i of the op); its op
    // index is 1 + NT l + k.  The prefixes live in registers and the division is a
    // multiply-high, so an item is located without dependent LDS reads.
    const int total = s_total;
    const int ipl = s_pre[NT];                  // items per layer (> 0 when total > 0)
    int pre[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) pre[k] = s_pre[k];
    const unsigned ipl_magic = ipl > 1 ? (unsigned)((0x100000000ULL + (unsigned)ipl - 1) / (unsigned)ipl) : 0u;
    struct ItemLoc {
        int l, k, i, ch, tl;
    };
    // DMA of attention item i of this workgroup's unit (layer lp) to LDS dst
    auto dma_attn = [&](const LayerPtrs &lp, int i, uint32_t dst) __attribute__((always_inline)) {
        const uint32_t d1 = dst + 1024, d2 = dst + 2048, d3 = dst + 3072, d4 = dst + 4096;
        // 8 cached keys: K rows [kb, kb + 8) (D 2 bytes each, from the slot's start; row r's
        // 16-byte chunks rotated by r, so the 8 rows' same chunk sits in different banks)
        // and V^T columns (D x 16 B, from byte 2048).  head_dim 64 fills half of each;
        // the other instructions reload the same bytes, so every item issues five.
        const int kb = au.lo + 8 * i;
        const uint8_t *kp = reinterpret_cast<const uint8_t *>(lp.kc + ((size_t)au.kvh * a.T_cap + kb) * D);
        const uint16_t *vp = lp.vt + (size_t)au.kvh * D * a.T_cap + kb;
        if (D == 128) {
            const int kr0 = lane >> 4, kr1 = 4 + (lane >> 4);
            dma16(kp + kr0 * 256 + (((lane & 15) + kr0) & 15) * 16, dst);
            dma16(kp + kr1 * 256 + (((lane & 15) + kr1) & 15) * 16, d1);
            dma16(vp + (size_t)lane * a.T_cap, d2);
            dma16(vp + (size_t)(64 + lane) * a.T_cap, d3);
        } else {
            const int kr = lane >> 3;
            dma16(kp + kr * 128 + (((lane & 7) + kr) & 7) * 16, dst);
            dma16(kp + kr * 128 + (((lane & 7) + kr) & 7) * 16, dst);
            dma16(vp + (size_t)lane * a.T_cap, d2);
            dma16(vp + (size_t)lane * a.T_cap, d2);
        }
        if (lane < 32) dma16(kp + 16 * lane, d4);
    };
    // DMA of item g to LDS dst: 4 weight instructions + 1 scale/bias (or 4 key/value + 1
    // filler) instructions.
    auto dma_item = [&](int g, uint32_t dst) __attribute__((always_inline)) -> ItemLoc {
        ItemLoc w;
        w.l = ipl == 1 ? g : (int)__umulhi((unsigned)g, ipl_magic);     // g * ipl < 2^32
        const int r = g - w.l * ipl;
        int kind = 0, base_k = 0;
#pragma unroll
        for (int kk = 1; kk < NT; ++kk)
            if (r >= pre[kk]) {
                kind = kk;
                base_k = pre[kk];
            }
        w.k = kind;
        w.i = r - base_k;
        w.ch = 0;
        w.tl = 0;
        const LayerPtrs &lp = slp[w.l];
        const uint32_t d1 = dst + 1024, d2 = dst + 2048, d3 = dst + 3072, d4 = dst + 4096;
        if (w.k != K_ATTN) {
            const int gi = gemv_index(w.k);
            const GemvDesc &o = sgd[gi];
            const int cpt = o.cpt;
            const int tl = cpt == 1 ? w.i : (int)__umulhi((unsigned)w.i, o.cpt_magic);
            const int ch = w.i - tl * cpt;
            w.ch = ch;
            w.tl = tl;
            const int n0 = o.rb + tl * 16;             // this workgroup's rows [o.rb, o.re)
            const int rlast = o.re - 1;
            const uint32_t row_bytes = (uint32_t)o.K * BITS / 8;        // every weight matrix < 4 GB
            const bool swiglu = o.flags & F_SWIGLU;
            const int half = o.half;
            const uint32_t G = (uint32_t)o.G;
            auto wrow = [&](int rr) -> uint32_t {
                if (swiglu) return (uint32_t)((rr < 8 ? 0 : half - 8) + (n0 >> 1) + rr);
                return (uint32_t)min(n0 + rr, rlast);
            };
            const uint8_t *wq = reinterpret_cast<const uint8_t *>(lp.wq[gi]) + ch * 256;
            const uint32_t dq[4] = {dst, d1, d2, d3};
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int rr = 4 * q4 + (lane >> 4);
                const int col = ((lane & 15) - rr) & 15;
                dma16(wq + (wrow(rr) * row_bytes + (uint32_t)(col * 16)), dq[q4]);
            }
            if (lane < 32)
                dma16((lane < 16 ? lp.s[gi] : lp.b[gi]) + (wrow(lane & 15) * G + (uint32_t)((ch * ITEM_GROUPS) & ~7)), d4);
        } else {
            dma_attn(lp, w.i, dst);
        }
        return w;
    };

    // ---- attention item: 8 keys of kv head au.kvh against its R query heads, on MFMA
    //   S^T[16 key rows (8 used) x 16 head columns (R used)] = K . Q^T   (4 x 16x16x32)
    //   p = exp2(S^T scale - max), per head over the 8 keys (fp32; l sums fp32 p)
    //   O^T[D x 16 heads] = V^T[D x keys] . P^T with P in bf16     (8 x 16x16x32)
    // as the per-op attention kernel computes a block.  The item's (m, l, O) per head
    // goes to state block i ([RMAX][D + 4] floats); the op's epilogue merges the
    // blocks in item order, so the sums do not depend on which wave took which item.
    // sl: the item's bytes in LDS (a worker's ring slot, or the control wave's item
    // area).  ac: MFMA column (key row of A, head column of B), ag: its k group.
    auto attn_compute = [&](int i, const uint8_t *sl) {
        const int R = a.R;
        // recomputed per item: hoisted out of the item loop, the per-tile addresses
        // would be held (and spilled) across the whole stream
        int ac = lane & 15;
        asm volatile("" : "+v"(ac));
        const int ag = lane >> 4;
        float *stw = ast + i * AST;
        const int kb = au.lo + 8 * i;
        const int nval = min(8, au.hi - kb);               // valid keys of the block, wave-uniform
        const int newk = T - 1 - kb;                       // the new key's slot in the block, if 0..7
        const bool has_new = newk >= 0 && newk < 8;        // wave-uniform
        // operand A: key row ac, chunk 4u + ag (cached row r's chunk c sits at slot
        // (c - r) & 15; rows 8..15 read the block's V^T bytes: their S rows are
        // masked, and MFMA rows do not mix).  The new key is not in the cache yet:
        // its rotated copy is in LDS.  Operand B: query head min(ac, R - 1), the same
        // chunk (columns past R are ignored).
        const uint4 *krow = reinterpret_cast<const uint4 *>(sl + ac * (2 * D));
        const uint4 *qrow = reinterpret_cast<const uint4 *>(qkv_l + min(ac, R - 1) * D);
        uint4 kv[D / 32], qv[D / 32];
#pragma unroll
        for (int u = 0; u < D / 32; ++u) {
            kv[u] = krow[(4 * u + ag - ac) & (KCH - 1)];
            qv[u] = qrow[4 * u + ag];
        }
        if (has_new) {
            const uint4 *knew = reinterpret_cast<const uint4 *>(qkv_l + RMAX * D);
#pragma unroll
            for (int u = 0; u < D / 32; ++u) {
                const uint4 kn = knew[4 * u + ag];
                if (ac == newk) kv[u] = kn;
            }
        }
        // V^T rows (dim 16 n + ac, keys 0..7): read now, so the reads overlap S and the softmax
        const uint4 *vrow = reinterpret_cast<const uint4 *>(sl + 2048 + ac * 16);
        uint4 vv[D / 16];
#pragma unroll
        for (int n = 0; n < D / 16; ++n) vv[n] = vrow[16 * n];
        f4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < D / 32; ++u)
            st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kv[u]), as_bf16x8(qv[u]), st, 0, 0, 0);
        // lane (ac = head, ag): keys 4 ag + r; keys 0-3 in lanes 0-15, 4-7 in lanes 16-31
        float sv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[r] = (4 * ag + r < nval) ? st[r] * a.scale_log2 : -INFINITY;
        float bm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        float x0, x1;
        swap16(bm, x0, x1);
        bm = fmaxf(x0, x1);                                // rows 0, 1: the max over the 8 keys
        float pv[4], ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pv[r] = (sv[r] == -INFINITY) ? 0.f : exp2f(sv[r] - bm);
            ps += pv[r];
        }
        swap16(ps, x0, x1);
        ps = x0 + x1;
        // operand B of O^T: lane (head ac, k group 0) holds keys 0..7 as bf16, the
        // other k groups zero
        float pk[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) swap16(pv[r], pk[r], pk[4 + r]);
        uint4 pw = make_uint4(cvt_pk_bf16(pk[0], pk[1]), cvt_pk_bf16(pk[2], pk[3]), cvt_pk_bf16(pk[4], pk[5]),
                              cvt_pk_bf16(pk[6], pk[7]));
        if (ag != 0) pw = make_uint4(0u, 0u, 0u, 0u);
        const bf16x8_t pb8 = as_bf16x8(pw);
        // operand A of O^T: V^T row (dim 16 n + ac) over keys 0..7 for k group 0, zero
        // for the others (their B is zero, and a zero A keeps them finite).  Block
        // with the new key: its value comes from LDS; keys past the range are zeroed
        // (their p is 0; cache slots past the length may hold anything).
        // lanes of k groups 1..3 are zeroed with a register mask, not a branch: a
        // branch over an operand with its LDS read in flight waits for that read, and
        // the eight reads of the block then run one after another
        uint32_t lm = ag == 0 ? 0xFFFFFFFFu : 0u;
        asm volatile("" : "+v"(lm));
        if (!has_new && nval == 8) {
            f4 o[D / 16];
#pragma unroll
            for (int n = 0; n < D / 16; ++n) {
                vv[n] = make_uint4(vv[n].x & lm, vv[n].y & lm, vv[n].z & lm, vv[n].w & lm);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vv[n]), pb8, f4{0.f, 0.f, 0.f, 0.f}, 0,
                                                               0, 0);
            }
            // lane (head ac, ag): dims 16 n + 4 ag + r
            if (ac < R)
#pragma unroll
                for (int n = 0; n < D / 16; ++n) *reinterpret_cast<f4 *>(stw + ac * (D + 4) + 16 * n + 4 * ag) = o[n];
        } else {
            uint32_t km[4];                                // per word: its elements < nval
#pragma unroll
            for (int w = 0; w < 4; ++w)
                km[w] = (nval >= 2 * w + 2 ? 0xFFFFFFFFu : nval == 2 * w + 1 ? 0x0000FFFFu : 0u) & lm;
            uint32_t nm[4];                                // per word: the new key's half
#pragma unroll
            for (int w = 0; w < 4; ++w) nm[w] = (has_new && (newk >> 1) == w) ? (0xFFFFu << ((newk & 1) * 16)) : 0u;
            const int nsh = (newk & 1) * 16;
            const uint16_t *vnew = qkv_l + RMAX * D + D + ac;
            uint32_t nv[D / 16];
#pragma unroll
            for (int n = 0; n < D / 16; ++n) nv[n] = (uint32_t)vnew[16 * n] << nsh;
#pragma unroll
            for (int n = 0; n < D / 16; ++n) {
                uint4 v = vv[n];
                v.x = ((v.x & ~nm[0]) | (nv[n] & nm[0])) & km[0];
                v.y = ((v.y & ~nm[1]) | (nv[n] & nm[1])) & km[1];
                v.z = ((v.z & ~nm[2]) | (nv[n] & nm[2])) & km[2];
                v.w = ((v.w & ~nm[3]) | (nv[n] & nm[3])) & km[3];
                const f4 o = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(v), pb8, f4{0.f, 0.f, 0.f, 0.f},
                                                                     0, 0, 0);
                if (ac < R) *reinterpret_cast<f4 *>(stw + ac * (D + 4) + 16 * n + 4 * ag) = o;
            }
        }
        if (ac < R && ag == 0) {
            stw[ac * (D + 4) + D] = bm;
            stw[ac * (D + 4) + D + 1] = ps;
        }
    };

    if (wave == CTL) {
        const uint8_t *own = smem + (ctl_item ? a.o_spare : 0);
        for (int jj = 0; jj <= nops; ++jj) {
            boundary(jj, std::true_type{});
            if (D == 128 && ctl_item && jj >= 1 && jj < nops && !s_abort) {
                // the x area past q|k|v's input and the attention states is free from
                // q|k|v's staging (the previous layer's down input is dead) until this
                // layer's attention items are merged
                const int k = kind_of(jj);
                if (k == K_QKV) {
                    dma_attn(slp[(jj - 1) / NT], ni_unit - 1, (uint32_t)(uintptr_t)own);
                } else if (k == K_ATTN) {
                    wait_vm<0>();
                    attn_compute(ni_unit - 1, own);
                }
            }
            const int kj = jj >= 1 && jj < nops ? kind_of(jj) : -1;
            // the attention items' merge weights, once the workers' items are counted
            if (kj == K_ATTN && ni_unit > 0 && !s_abort) {
                const int nw = ni_unit - (ctl_item ? 1 : 0);
                bool ready = true;
                for (int it = 0;
                     __hip_atomic_load(&s_tile[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < nw; ++it) {
                    if (s_abort || ((it & 255) == 255 && expired())) {
                        ready = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                if (ready) {
                    const int ni = ni_unit;
                    float *fac = part, *mh = part + a.R * ni;
                    for (int t = lane; t < a.R * ni; t += 64) {
                        const int h = t / ni, w = t - h * ni;
                        const float *mrow = ast + h * (D + 4) + D;
                        float M = -INFINITY;
                        for (int v = 0; v < ni; ++v) M = fmaxf(M, mrow[v * AST]);
                        const float mw = mrow[w * AST];
                        fac[t] = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
                        if (w == 0) mh[h] = M;
                    }
                }
            }
            // a projection's tiles published as the workers complete them (all of a tile's
            // K chunks counted), so that the op boundary finds them out already
            if ((kj == K_QKV || kj == K_O || kj == K_GU || kj == K_DOWN) && !s_abort) {
                const GemvDesc &o = sgd[gemv_index(kj)];
                if (o.ntl <= MAX_TILES) {
                    const uint32_t ep = epoch(jj);
                    const int lj = (jj - 1) / NT;
                    int t0 = 0;
                    for (int it = 0; t0 < o.ntl; ++it) {
                        int t1 = t0;
                        while (t1 < o.ntl &&
                               __hip_atomic_load(&s_tile[t1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) ==
                                   o.cpt)
                            ++t1;
                        if (t1 > t0) {
                            __builtin_amdgcn_s_setprio(3);
                            publish_tiles(kj, lj, ep, t0, t1);
                            __builtin_amdgcn_s_setprio(0);
                            t0 = t1;
                            continue;
                        }
                        // polled without a sleep (measured: TinyLlama 0.4 % faster, 8B the same);
                        // a launch that gives up here records it and stops every wave
                        if (s_abort) break;
                        if ((it & 255) == 255 && timed_out()) {
                            if (lane == 0) s_abort = 1;
                            break;
                        }
                    }
                    if (t0 == o.ntl) early_done = jj;
                }
            }
        }
        wait_vm<0>();                                   // no DMA may land after the workgroup ends
        if (lane == 0 && s_abort) atomicOr(a.status, 2u);
        if (wg == 0 && lane == 0) {
            // every workgroup read the base before producing anything, and workgroup 0
            // ends after consuming every workgroup's outputs of the last gate|up
            a.epoch_base[0] = base + 1u;
        }
        return;
    }

    {
        // ================================================================ worker
        uint8_t *ring = smem + (size_t)wave * TRING * SLOT;
        const uint32_t ring_lds = (uint32_t)(uintptr_t)ring;

        // per ring slot: op index, op kind, item of the op, and (projections) its K chunk
        // and tile
        int sj[TRING], sk[TRING], si[TRING], sch[TRING], stl[TRING];
        // DMA of item g into ring slot `slot`
        auto issue = [&](int g, int slot) {
            const ItemLoc w = dma_item(min(g, total - 1), ring_lds + slot * SLOT);
            sj[slot] = 1 + NT * w.l + w.k;
            sk[slot] = w.k;
            si[slot] = w.i;
            sch[slot] = w.ch;
            stl[slot] = w.tl;
        };

        // ---- projection item (the math of qgemv_m1_kernel)
        const int j16 = lane & 15, q = lane >> 4;
        const bool a_zero = BITS == 4 && ((j16 == 0 && q >= 2) || (j16 == 8 && q < 2));
        const int epar = BITS == 4 ? (q >> 1) : 0;
        const int xq = BITS == 4 ? 4 * q : 2 * q;
        uint32_t magic = 0x43004300u;
        asm volatile("" : "+v"(magic));
        uint32_t nib_mask = 0x000F000Fu;
        asm volatile("" : "+s"(nib_mask));

        auto gemv_item = [&](int ch, int i, int slot) {
            const uint4 *sl = reinterpret_cast<const uint4 *>(ring + slot * SLOT);
            uint4 wv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) wv[t] = sl[(j16 >> 2) * 64 + (j16 & 3) * 16 + ((4 * t + q + j16) & 15)];
            const uint4 sv = sl[4096 / 16 + j16];
            const uint4 bv = sl[4096 / 16 + 16 + j16];
            const int gsub = (ch * ITEM_GROUPS) & 7;
            const uint4 *xrow = a_zero ? xzero : xl + ch * 4 * SPAN_WORDS;
            float xsv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) xsv[t] = xs[(ch * 4 + t) * SPAN_GROUPS + epar];
            f4 P4[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) P4[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < MFMAS; ++u) {
                // x for this step of the four chains (loaded per step: registers are short)
                uint4 xa[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) xa[t] = xrow[t * SPAN_WORDS + xq + u];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    bf16x8_t Bv;
                    if (BITS == 4) {
                        const uint32_t w = wc(wv[t], u);
                        Bv = as_bf16x8(and_or(w, nib_mask, magic), and_or(w >> 4, nib_mask, magic),
                                       and_or(w >> 8, nib_mask, magic), and_or(w >> 12, nib_mask, magic));
                    } else {
                        const uint32_t w0 = wc(wv[t], 2 * u), w1 = wc(wv[t], 2 * u + 1);
                        Bv = as_bf16x8(byte_pair_lo(w0), byte_pair_hi(w0), byte_pair_lo(w1), byte_pair_hi(w1));
                    }
                    P4[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[t]), Bv, P4[t], 0, 0, 0);
                }
            }
            float acc = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int gsel = gsub + t * SPAN_GROUPS + epar;
                const float sf = bf2f(wh(sv, gsel));
                const float bf = bf2f(wh(bv, gsel));
                const float cf = BITS == 4 ? fmaf(-128.f, sf, bf) : bf;
                acc = fmaf(sf, P4[t][0], fmaf(cf, xsv[t], acc));
            }
            if (BITS == 4) acc = xor32_sum(acc);
            if (q == 0) part[i * 16 + j16] = acc;
        };

        auto attn_item = [&](int i, int slot) { attn_compute(i, ring + slot * SLOT); };

        // Every op boundary up to and including op k's staging, before the item of op
        // k is awaited: the other waves need not wait for this wave's next DMA.
        int staged = 0;
        auto catch_up = [&](int k) __attribute__((always_inline)) {
            while (staged <= k) {
                boundary(staged, std::false_type{});
                ++staged;
            }
        };
        auto compute = [&](int slot) {
            if (sk[slot] == K_ATTN) attn_item(si[slot], slot);
            else gemv_item(sch[slot], si[slot], slot);
        };
        auto claim = [&]() -> int {
            int v = 0;
            if (lane == 0) v = atomicAdd(&s_ctr, 1);
            return __builtin_amdgcn_readfirstlane(v);
        };

        if (total > 0) {
            // slot s holds item held[s]; TRING - 1 items in flight while one is computed
            int held[TRING];
#pragma unroll
            for (int s = 0; s < TRING - 1; ++s) {
                held[s] = wave + WORKERS * s;
                issue(held[s], s);
            }
            bool more = true;
            while (more) {
#pragma unroll
                for (int s = 0; s < TRING; ++s) {
                    if (more) {
                        const int nx = (s + TRING - 1) % TRING;
                        held[nx] = claim();
                        issue(held[nx], nx);
                        if (held[s] >= total) {
                            more = false;
                        } else {
                            catch_up(sj[s]);
                            if (s_abort) {
                                more = false;
                            } else {
                                wait_vm<DMA_PER_ITEM * (TRING - 1)>();
                                compute(s);
                                // the item's partials (or attention state) are in LDS: count
                                // it for its tile (attention: tile 0; the release orders this
                                // wave's LDS writes before the count)
                                if (stl[s] < MAX_TILES && lane == 0)
                                    __hip_atomic_fetch_add(&s_tile[stl[s]], 1, __ATOMIC_RELEASE,
                                                           __HIP_MEMORY_SCOPE_WORKGROUP);
                            }
                        }
                    }
                }
            }
        }
        catch_up(nops);                                 // the remaining boundaries, the last one finishing the step
        wait_vm<0>();                                   // no DMA may land after the workgroup ends
    }
}

// ---------------------------------------------------------------- host side

struct DecodePlan {
    int device = 0;
    int bits = 4;
    int head_dim = 128;         // with RMAX 4 (128) or 8 (64)
    int P = 0;
    Args args{};
    LayerPtrs *d_layers = nullptr;
    void *d_mem = nullptr;      // exchange buffers, epoch base, status
    uint32_t *d_trace = nullptr;  // op timeline (allocated while tracing)
    size_t lds = 0;
};

static size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

int decode_plan_create(const sc_decode_model *m, const sc_decode_layer *layers, void **out) {
    if (!m || !layers || !out) return set_error(SC_EINVAL, "decode_plan: null argument");
    *out = nullptr;
    const int L = m->num_layers, hid = m->hidden, I = m->intermediate, H = m->num_heads, Hkv = m->num_kv_heads,
              D = m->head_dim;
    if (m->bits != 4 && m->bits != 8) return set_error(SC_EUNSUPPORTED, "decode_plan: bits must be 4 or 8");
    if (m->group_size != 64) return set_error(SC_EUNSUPPORTED, "decode_plan: group size 64 only");
    if (D != 128 && D != 64) return set_error(SC_EUNSUPPORTED, "decode_plan: head_dim %d (64 or 128)", D);
    // query heads per kv head: up to 4 at head_dim 128, up to 8 at 64 (the kernels built)
    const int RMAX = D == 128 ? 4 : 8;
    if (L <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || H / Hkv > RMAX)
        return set_error(SC_EUNSUPPORTED, "decode_plan: at most %d query heads per kv head at head_dim %d", RMAX, D);
    if (hid % 512 || I % 512 || (H * D) % 512)
        return set_error(SC_EUNSUPPORTED, "decode_plan: widths must be multiples of 512");
    if (hid > 16384 || I > 16384 || H * D > 16384)
        return set_error(SC_EUNSUPPORTED, "decode_plan: widths up to 16384");
    if (m->T_cap <= 0 || m->T_cap % 32) return set_error(SC_EINVAL, "decode_plan: cache capacity must be a multiple of 32");
    if (!m->counters || !m->ids || !m->embed || !m->cos_t || !m->sin_t || !m->h_out)
        return set_error(SC_EINVAL, "decode_plan: null model pointer");
    if (m->vocab_local <= 0 || m->vocab_local >= (1L << 31) || m->table_len <= 0 || m->pos_offset < 0)
        return set_error(SC_EINVAL, "decode_plan: bad vocabulary or rotary table");
    int dev = 0;
    SC_HIP_CHECK(hipGetDevice(&dev));
    const DeviceInfo &di = device_info();
    // Workgroups: one per CU, or one per two CUs for layers of under 32 MB of weights,
    // whose ops are short enough that the op boundaries, not the weight stream, set
    // the step (TinyLlama's 22 MB layers: 0.80 -> 0.75 ms per step on half the CUs;
    // the Llama-3-8B's 109 MB layers need every CU's share of HBM).
    const double layer_bytes = ((double)qkv_rows(H, Hkv, D) * hid + (double)hid * H * D + 2.0 * I * hid +
                                (double)hid * I) * m->bits / 8;
    int P = di.num_cus;
    // half the CUs when the merge of the attention rows still splits evenly over them
    // (the same conditions as below, at twice the rows per workgroup)
    auto merge_ok = [&](int p) {
        const int c = p > 0 && (H * D) % p == 0 ? (H * D) / p : 0;
        return c >= 2 && c % 2 == 0 && c <= 32 && D % c == 0 && p / Hkv >= 1;
    };
    if (layer_bytes < 32e6 && P % 2 == 0 && merge_ok(P / 2)) P /= 2;
    if (P < 8 || P > 4096) return set_error(SC_EUNSUPPORTED, "decode_plan: %d CUs", P);
    const int R = H / Hkv;
    const int NR = P / Hkv;
    if (NR < 1 || NR > 64) return set_error(SC_EUNSUPPORTED, "decode_plan: %d kv heads on %d CUs", Hkv, P);
    const int C = (H * D) / P;
    if ((H * D) % P || C < 2 || C % 2 || C > 32 || D % C)
        return set_error(SC_EUNSUPPORTED, "decode_plan: attention rows do not split over %d CUs", P);
    const int qkvN = (H + 2 * Hkv) * D;

    Args a{};
    auto desc = [&](int N, int K, int flags, int in_buf, int out_buf) {
        GemvDesc g{};
        g.N = N; g.K = K; g.G = K / 64;
        g.T = (flags & F_SWIGLU) ? N / 16 : (N + 15) / 16;
        g.cpt = K / (m->bits == 4 ? 512 : 256);
        g.cpt_magic = g.cpt > 1 ? (unsigned)((0x100000000ULL + (unsigned long long)g.cpt - 1) / (unsigned long long)g.cpt) : 0u;
        g.half = (flags & F_SWIGLU) ? N / 2 : 0;
        // 8-row ranges when they lower the most rows a workgroup owns (gemv_rows)
        if (!(flags & F_SWIGLU) && ((N + 7) / 8 + P - 1) / P * 8 < (g.T + P - 1) / P * 16) flags |= F_ROW8;
        g.flags = flags; g.in_buf = in_buf; g.out_buf = out_buf;
        return g;
    };
    a.gd[0] = desc(qkvN, hid, F_NORM, B_H, B_QKV);
    a.gd[1] = desc(hid, H * D, F_RESID, B_ATT, B_HMID);
    a.gd[2] = desc(2 * I, hid, F_NORM | F_SWIGLU, B_HMID, B_ACT);
    a.gd[3] = desc(hid, I, F_RESID, B_ACT, B_H);

    std::vector<LayerPtrs> lps(L);
    for (int l = 0; l < L; ++l) {
        const sc_decode_layer &y = layers[l];
        LayerPtrs &p = lps[l];
        p.wq[0] = y.wq_qkv; p.s[0] = y.s_qkv; p.b[0] = y.b_qkv;
        p.wq[1] = y.wq_o; p.s[1] = y.s_o; p.b[1] = y.b_o;
        p.wq[2] = y.wq_gu; p.s[2] = y.s_gu; p.b[2] = y.b_gu;
        p.wq[3] = y.wq_down; p.s[3] = y.s_down; p.b[3] = y.b_down;
        p.ln[0] = y.ln_in; p.ln[1] = y.ln_post;
        p.kc = y.kc; p.vt = y.vt;
        for (int i = 0; i < 4; ++i)
            if (!p.wq[i] || !p.s[i] || !p.b[i] || (((uintptr_t)p.wq[i] | (uintptr_t)p.s[i] | (uintptr_t)p.b[i]) % 16))
                return set_error(SC_EINVAL, "decode_plan: layer %d: null or misaligned weights", l);
        if (!p.ln[0] || !p.ln[1] || (((uintptr_t)p.ln[0] | (uintptr_t)p.ln[1]) % 16) || !p.kc || !p.vt ||
            (((uintptr_t)p.kc | (uintptr_t)p.vt) % 16))
            return set_error(SC_EINVAL, "decode_plan: layer %d: null or misaligned norm/cache pointers", l);
    }

    // LDS layout
    const int Kmax = std::max({hid, I, H * D});
    int max_items = 0;
    for (int i = 0; i < 4; ++i) {
        const GemvDesc &g = a.gd[i];
        const int tiles = (g.flags & F_ROW8) ? (((g.N + 7) / 8 + P - 1) / P + 1) / 2 : (g.T + P - 1) / P;
        max_items = std::max(max_items, tiles * g.cpt);
    }
    // attention item states: ceil(keys per unit / 8) blocks of RMAX (D + 4) floats
    const int kps_max = ((m->T_cap + NR - 1) / NR + 7) & ~7;
    const int n_items = kps_max / 8;            // attention items per unit at most
    const size_t item_state = (size_t)RMAX * (D + 4) * 4;
    const size_t ast_bytes = (size_t)n_items * item_state;
    const int lds_cap = di.max_lds_per_block < 160 * 1024 ? di.max_lds_per_block : 160 * 1024;
    // the layout for an x area of xarea bytes (which the attention states overlay) and
    // merge weights for up to fac_items items per unit; returns the bytes used
    auto layout = [&](size_t xarea, int fac_items) -> size_t {
        size_t o = (size_t)WORKERS * TRING * SLOT;
        a.o_xl = (int)o; o += xarea;
        a.o_xzero = (int)o; o += 1024;
        a.o_xs = (int)o; o += align16((size_t)(Kmax / 64) * 4);
        // projection partials (16 floats per item), or the attention items' merge
        // weights [R][items] and maxima [R]
        a.o_part = (int)o;
        o += align16(std::max((size_t)max_items * 64, ((size_t)RMAX * fac_items + RMAX) * 4));
        a.o_hbuf = (int)o; o += align16((size_t)hid * 2);
        a.o_qkv = (int)o; o += align16((size_t)(RMAX + 2) * D * 2);
        a.o_gd = (int)o; o += align16(4 * sizeof(GemvDesc));
        a.o_lp = (int)o; o += (size_t)L * sizeof(LayerPtrs);
        return o;
    };
    size_t xarea = align16(std::max((size_t)Kmax * 2, ast_bytes));
    size_t off = layout(xarea, n_items);
    if (off + 512 > (size_t)lds_cap)                 // + the kernel's static LDS (under 512 bytes)
        return set_error(SC_EUNSUPPORTED, "decode_plan: needs %zu bytes of LDS (limit %d)", off, lds_cap);
    // One key range per kv head for contexts up to 8 x single_items positions (at most
    // 8 items, one round of the workers: with 16, TinyLlama was 0.8 % slower than with
    // the ranges and their merge), the x area grown into the LDS left over to hold
    // their states.  head_dim 64 only.  SC_TRUNK_SINGLE_RANGE=0 at plan creation turns
    // it off.
    int single_items = 0;
    {
        const char *ev = getenv("SC_TRUNK_SINGLE_RANGE");
        if (D == 64 && !(ev && ev[0] == '0')) {
            for (int si = 8; si >= 1; --si) {
                const size_t xa = align16(std::max(xarea, (size_t)si * item_state));
                if (layout(xa, std::max(n_items, si)) + 512 <= (size_t)lds_cap) {
                    single_items = si;
                    xarea = xa;
                    break;
                }
            }
        }
        off = layout(xarea, std::max(n_items, single_items));
    }
    a.single_max = 8 * single_items;
    // the control wave's attention item (one ring slot), in the x area past q|k|v's
    // input and the attention states, when it fits there.  SC_TRUNK_CONTROL_ITEM=0 in
    // the environment at plan creation leaves every item to the workers (the results
    // are the same bits: the states merge in item order whoever computed them).
    {
        const size_t rel = align16(std::max(ast_bytes, (size_t)hid * 2));
        a.o_spare = rel + SLOT <= xarea ? (int)(a.o_xl + rel) : -1;
        const char *ev = getenv("SC_TRUNK_CONTROL_ITEM");
        if (ev && ev[0] == '0') a.o_spare = -1;
    }
    a.lds_bytes = (int)off;

    // device memory: layer table, exchange buffers, epoch base, status
    const size_t nb_h = (size_t)hid / 2, nb_qkv = (size_t)qkvN / 2, nb_part = (size_t)Hkv * NR * R * (D + 2),
                 nb_att = (size_t)H * D / 2, nb_act = (size_t)I / 2;
    const size_t words[B_COUNT] = {nb_h, nb_qkv, nb_part, nb_att, nb_h, nb_act};
    size_t mem = 256;
    size_t boff[B_COUNT];
    for (int i = 0; i < B_COUNT; ++i) {
        boff[i] = mem;
        mem += ((words[i] * 8 + 255) / 256) * 256;
    }
    std::unique_ptr<DecodePlan> pl(new DecodePlan());
    pl->device = dev;
    pl->bits = m->bits;
    pl->head_dim = D;
    pl->P = P;
    pl->lds = off;
    SC_HIP_CHECK(hipMalloc(&pl->d_mem, mem));
    SC_HIP_CHECK(hipMemset(pl->d_mem, 0, mem));
    SC_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&pl->d_layers), (size_t)L * sizeof(LayerPtrs)));
    SC_HIP_CHECK(hipMemcpy(pl->d_layers, lps.data(), (size_t)L * sizeof(LayerPtrs), hipMemcpyHostToDevice));
    uint8_t *mb = static_cast<uint8_t *>(pl->d_mem);
    const uint32_t one = 1;
    SC_HIP_CHECK(hipMemcpy(mb, &one, 4, hipMemcpyHostToDevice));   // epoch base starts at 1
    a.layers = pl->d_layers;
    for (int i = 0; i < B_COUNT; ++i) a.buf[i] = reinterpret_cast<uint2 *>(mb + boff[i]);
    for (int i = 0; i < 4; ++i) {
        a.gd[i].in = a.buf[a.gd[i].in_buf];
        a.gd[i].out = a.buf[a.gd[i].out_buf];
    }
    a.counters = m->counters;
    a.epoch_base = reinterpret_cast<uint32_t *>(mb);
    a.status = reinterpret_cast<unsigned *>(mb + 64);
    a.ids = m->ids;
    a.embed = m->embed;
    a.cos_t = m->cos_t;
    a.sin_t = m->sin_t;
    a.h_out = m->h_out;
    a.vocab_start = m->vocab_start;
    a.V_local = (int)m->vocab_local;
    a.table_len = m->table_len;
    a.pos_offset = m->pos_offset;
    a.L = L;
    a.nops = 1 + NT * L;
    a.hidden = hid;
    a.H = H; a.Hkv = Hkv; a.R = R; a.NR = NR; a.T_cap = m->T_cap;
    a.C_merge = C;
    a.eps = m->eps;
    a.scale_log2 = m->scale * 1.4426950408889634f;
    pl->args = a;
    SC_HIP_CHECK(hipDeviceSynchronize());
    *out = pl.release();
    return SC_OK;
}

int decode_plan_run(void *plan, hipStream_t stream) {
    DecodePlan *pl = static_cast<DecodePlan *>(plan);
    if (!pl) return set_error(SC_EINVAL, "decode_plan_run: null plan");
    int dev = 0;
    SC_HIP_CHECK(hipGetDevice(&dev));
    if (dev != pl->device) return set_error(SC_EINVAL, "decode_plan_run: plan belongs to device %d", pl->device);
    auto go = [&](auto kern, int variant) -> int {
        static int configured[4] = {0, 0, 0, 0};
        int &cfg = configured[variant];
        if ((int)pl->lds > cfg) {
            SC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl->lds));
            cfg = (int)pl->lds;
        }
        int occ = 0;
        SC_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void *>(kern), THREADS,
                                                                  pl->lds));
        if (occ < 1) return set_error(SC_EUNSUPPORTED, "decode_plan_run: kernel does not fit on a CU");
        hipLaunchKernelGGL(kern, dim3(pl->P), dim3(THREADS), pl->lds, stream, pl->args);
        SC_HIP_CHECK(hipGetLastError());
        return SC_OK;
    };
    if (pl->head_dim == 128) {
        if (pl->bits == 4) return go(decode_step_kernel<4, 128, 4>, 0);
        return go(decode_step_kernel<8, 128, 4>, 1);
    }
    if (pl->bits == 4) return go(decode_step_kernel<4, 64, 8>, 2);
    return go(decode_step_kernel<8, 64, 8>, 3);
}

int decode_plan_status(void *plan, unsigned *status) {
    DecodePlan *pl = static_cast<DecodePlan *>(plan);
    if (!pl || !status) return set_error(SC_EINVAL, "decode_plan_status: null argument");
    SC_HIP_CHECK(hipMemcpy(status, pl->args.status, 4, hipMemcpyDeviceToHost));
    return SC_OK;
}

int decode_plan_trace(void *plan, int enable) {
    DecodePlan *pl = static_cast<DecodePlan *>(plan);
    if (!pl) return set_error(SC_EINVAL, "decode_plan_trace: null plan");
    // The stamp buffer, once allocated, lives until sc_decode_plan_destroy: a graph
    // captured while tracing was on keeps writing stamps into it on every replay, also
    // after tracing is switched off for later launches.
    const size_t bytes = (size_t)pl->P * pl->args.nops * 4 * sizeof(uint32_t);
    if (enable && !pl->d_trace) {
        SC_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&pl->d_trace), bytes));
        SC_HIP_CHECK(hipMemset(pl->d_trace, 0, bytes));
    }
    pl->args.trace = enable ? pl->d_trace : nullptr;
    return SC_OK;
}

int decode_plan_read_trace(void *plan, uint32_t *host, int64_t n, int *P, int *nops) {
    DecodePlan *pl = static_cast<DecodePlan *>(plan);
    if (!pl || !P || !nops) return set_error(SC_EINVAL, "decode_plan_read_trace: null argument");
    *P = pl->P;
    *nops = pl->args.nops;
    if (!host) return SC_OK;
    if (!pl->d_trace) return set_error(SC_EINVAL, "decode_plan_read_trace: tracing was never enabled");
    const int64_t need = (int64_t)pl->P * pl->args.nops * 4;
    if (n < need) return set_error(SC_EINVAL, "decode_plan_read_trace: %lld entries needed", (long long)need);
    SC_HIP_CHECK(hipMemcpy(host, pl->d_trace, (size_t)need * sizeof(uint32_t), hipMemcpyDeviceToHost));
    return SC_OK;
}

void decode_plan_destroy(void *plan) {
    DecodePlan *pl = static_cast<DecodePlan *>(plan);
    if (!pl) return;
    if (pl->d_trace) (void)hipFree(pl->d_trace);
    (void)hipFree(pl->d_layers);
    (void)hipFree(pl->d_mem);
    delete pl;
}

}  // namespace sc
