// Decoder wiring kernels around the quantized linears: RMSNorm (with the
// residual add of the previous sub-block fused in), RoPE + KV-cache append,
// causal GQA attention on MFMA, SiLU-gate, greedy argmax and step counters.
//
// Every kernel that depends on the sequence position reads it from a device
// counter (the cache length) rather than from a launch argument, so a decode
// step captured once in a HIP graph replays correctly at every position.
//
// KV cache layout per layer (capacity T_cap, a multiple of 32):
//   K  [B, Hkv, T_cap, D]  keys in rows     (operand A of S^T = K Q^T)
//   Vt [B, Hkv, D, T_cap]  values transposed (operand A of O^T = Vt P^T)
#include "sc_common.h"

#include <math.h>
#include <float.h>

namespace sc {

namespace {

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f4;

}  // namespace

// ---------------------------------------------------------------- RMSNorm
//
// h = x (+ residual, rounded to bf16), y = (h / sqrt(mean(h*h) + eps)) * w
// (parallel/transformer.py:46-61; the residual add is transformer.py:246/252).
// One workgroup per row, up to MAXV uint4 per thread kept in registers.  The
// per-element arithmetic is IEEE single ops in the reference's order (divide by
// the root, then multiply by the weight); contraction to FMA is switched off in
// every kernel whose output is compared bit for bit.
constexpr int NORM_MAXV = 8;   // D <= 256 * 8 * 8 = 16384

__global__ void __launch_bounds__(NORM_THREADS)
add_rms_norm_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ res,
                    const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
                    uint16_t *__restrict__ h_out, int D, float eps) {
    const int row = blockIdx.x;
    const int nv = D >> 3;
    const uint4 *xr = reinterpret_cast<const uint4 *>(x + (size_t)row * D);
    const uint4 *rr = res ? reinterpret_cast<const uint4 *>(res + (size_t)row * D) : nullptr;
    const uint4 *wr = reinterpret_cast<const uint4 *>(w);
    // every load of the row (and of the weight) is issued before the first use: the
    // loads of a thread's chunks are independent, and one round trip to memory is
    // the kernel's main cost at decode sizes
    uint4 hv[NORM_MAXV], rv[NORM_MAXV], wv[NORM_MAXV];
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) {
        const int idx = threadIdx.x + i * NORM_THREADS;
        if (idx < nv) {
            hv[i] = xr[idx];
            if (rr) rv[i] = rr[idx];
            wv[i] = wr[idx];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) {
        const int idx = threadIdx.x + i * NORM_THREADS;
        if (idx < nv) {
            uint4 v = hv[i];
            if (rr) {
                v = add_bf16x8(v, rv[i]);
                if (h_out) reinterpret_cast<uint4 *>(h_out + (size_t)row * D)[idx] = v;
            }
            hv[i] = v;
            ss = sumsq_bf16x8(ss, v);
        }
    }
    __shared__ float red[NORM_THREADS / 64];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
    const float root = rms_root(tot, D, eps);
    uint4 *yr = reinterpret_cast<uint4 *>(y + (size_t)row * D);
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) {
        const int idx = threadIdx.x + i * NORM_THREADS;
        if (idx < nv) yr[idx] = norm_bf16x8(hv[i], wv[i], root);
    }
}

// The residual add and RMSNorm after a projection, with the projection's split-K
// pass folded in: y = bf16(sum over splits of partials [splits, rows, D], in split
// order) (+ bias, rounded again) -- or y read as bf16 when splits = 0 -- then
// h = bf16(y + res) and out = RMSNorm(h) * w, bit for bit launch_qmm_finalize followed
// by add_rms_norm_kernel (the sum of squares in that kernel's 256-thread partition).
// One workgroup per row, one thread per chunk of 8 up to 1024 threads (256 at least):
// all of a chunk's loads in flight together.  y_in may be `out` (each row is read
// whole before it is written).
constexpr int PNORM_THREADS = 1024;

__global__ void __launch_bounds__(PNORM_THREADS)
split_add_rms_norm_kernel(const float *partials, int splits, const uint16_t *y_in, const uint16_t *bias,
                          const uint16_t *res, const uint16_t *w, uint16_t *h_out, uint16_t *out, long rows, int D,
                          float eps) {
    __shared__ uint4 hs[NORM_THREADS * NORM_MAXV];
    __shared__ float red[NORM_THREADS / 64];
    const long row = blockIdx.x;
    const int nv = D >> 3;
    const size_t total = (size_t)rows * D;
    const int nt = blockDim.x;
    for (int c = threadIdx.x; c < nv; c += nt) {
        const size_t e0 = (size_t)row * D + 8 * (size_t)c;
        const uint4 r = reinterpret_cast<const uint4 *>(res + e0)[0];
        uint4 y;
        if (splits == 0) {
            y = reinterpret_cast<const uint4 *>(y_in + e0)[0];
        } else {
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            int sp = 0;
            for (; sp + 4 <= splits; sp += 4) {          // four splits' loads in flight
                float4 p[4][2];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 *src = reinterpret_cast<const float4 *>(partials + (size_t)(sp + u) * total + e0);
                    p[u][0] = src[0];
                    p[u][1] = src[1];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    v[0] += p[u][0].x; v[1] += p[u][0].y; v[2] += p[u][0].z; v[3] += p[u][0].w;
                    v[4] += p[u][1].x; v[5] += p[u][1].y; v[6] += p[u][1].z; v[7] += p[u][1].w;
                }
            }
            for (; sp < splits; ++sp) {
                const float4 *src = reinterpret_cast<const float4 *>(partials + (size_t)sp * total + e0);
                const float4 p0 = src[0], p1 = src[1];
                v[0] += p0.x; v[1] += p0.y; v[2] += p0.z; v[3] += p0.w;
                v[4] += p1.x; v[5] += p1.y; v[6] += p1.z; v[7] += p1.w;
            }
            uint32_t o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = f2bf(v[e]);
            if (bias) {
                const uint4 bb = reinterpret_cast<const uint4 *>(bias)[c];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = f2bf(bf2f(o[e]) + bfe(bb, e));
            }
            y = make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
        }
        const uint4 h = add_bf16x8(y, r);
        reinterpret_cast<uint4 *>(h_out + e0)[0] = h;
        hs[c] = h;
    }
    __syncthreads();
    if (threadIdx.x < NORM_THREADS) {
        float ss = 0.f;
        for (int c = threadIdx.x; c < nv; c += NORM_THREADS) ss = sumsq_bf16x8(ss, hs[c]);
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
    const float root = rms_root(tot, D, eps);
    for (int c = threadIdx.x; c < nv; c += nt)
        reinterpret_cast<uint4 *>(out + (size_t)row * D)[c] =
            norm_bf16x8(hs[c], reinterpret_cast<const uint4 *>(w)[c], root);
}

// ---------------------------------------------------------------- RoPE + KV append
//
// Token (b, s) goes to cache slot cache_len + s and is rotated for position
// cache_len + s + pos_offset (parallel/attention.py:421-427; the offset serves
// cache-less calls such as forward_sync_partial(position_offset=...)).
// q and k heads are rotated with the rotate-half rule x*cos + [-x2, x1]*sin
// (attention.py:130-151) using fp32 tables; rotated q is written back in place,
// rotated k and the raw v go to the cache.
// v_heads: Hkv (this kernel also appends v), or 0 when v_append_kernel does.
__global__ void __launch_bounds__(256)
rope_append_kernel(uint16_t *__restrict__ qkv, long qkv_stride, int S, int H, int Hkv, int D,
                   const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                   uint16_t *__restrict__ kc, uint16_t *__restrict__ vt, int T_cap,
                   const int32_t *__restrict__ cache_len, int pos_offset, int table_len, int v_heads) {
    // one wave per head of one token: q heads, then k heads, then v heads
    const int tok = blockIdx.x;
    const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (head >= H + Hkv + v_heads) return;
    const int b = tok / S, s = tok - (tok / S) * S;
    const int pos = cache_len[0] + s;             // cache slot
    const int rpos = pos + pos_offset;            // rotary position
    // the host sizes cache and tables for every launch; a counter that has run past
    // them (a stale replay) leaves the cache untouched instead of writing out of bounds
    if (pos < 0 || pos >= T_cap || rpos < 0 || rpos >= table_len) return;
    uint16_t *hp = qkv + (size_t)tok * qkv_stride + (size_t)head * D;
    const int half = D >> 1;
    if (head < H + Hkv) {
        const float *ct = cos_t + (size_t)rpos * half;
        const float *st = sin_t + (size_t)rpos * half;
        uint16_t *kr = kc + (((size_t)b * Hkv + (head - H)) * T_cap + pos) * D;
        for (int i = lane; i < half; i += 64) {
            const float x1 = bf2f(hp[i]), x2 = bf2f(hp[i + half]);
            const float c = ct[i], sn = st[i];
            const uint16_t o1 = (uint16_t)f2bf(add_rn(mul_rn(x1, c), mul_rn(-x2, sn)));
            const uint16_t o2 = (uint16_t)f2bf(add_rn(mul_rn(x2, c), mul_rn(x1, sn)));
            if (head < H) {
                hp[i] = o1;
                hp[i + half] = o2;
            } else {
                kr[i] = o1;
                kr[i + half] = o2;
            }
        }
    } else {
        const int hk = head - H - Hkv;
        uint16_t *vc = vt + ((size_t)b * Hkv + hk) * D * T_cap + pos;
        for (int d = lane; d < D; d += 64) vc[(size_t)d * T_cap] = hp[d];
    }
}

// The v part of rope_append for many new positions: Vt rows are [D, T_cap], so one
// token's values land in D different rows; a workgroup takes 64 tokens of one kv head
// through LDS and writes each dim's 64 consecutive slots with consecutive lanes
// (one-token-per-wave scattering makes every 2-byte store touch its own line).
// Same slots, same values, same bounds rule as rope_append_kernel.
constexpr int VAPP_TOK = 64;
__global__ void __launch_bounds__(256)
v_append_kernel(const uint16_t *__restrict__ qkv, long qkv_stride, int S, int H, int Hkv, int D,
                uint16_t *__restrict__ vt, int T_cap, const int32_t *__restrict__ cache_len, int pos_offset,
                int table_len) {
    __shared__ uint32_t tile[VAPP_TOK * (128 / 2 + 1)];   // token rows of D/2 + 1 words (odd: conflict-free columns)
    const int s0 = blockIdx.x * VAPP_TOK, hk = blockIdx.y, b = blockIdx.z;
    const int W = D / 2 + 1, cpt = D / 8;                  // words per LDS row, uint4 per token
    const int base = cache_len[0];
    for (int i = threadIdx.x; i < VAPP_TOK * cpt; i += 256) {
        const int t = i / cpt, c = i - t * cpt;
        if (s0 + t < S) {
            const uint4 v = *reinterpret_cast<const uint4 *>(qkv + (size_t)(b * S + s0 + t) * qkv_stride +
                                                             (size_t)(H + Hkv + hk) * D + 8 * c);
            uint32_t *row = tile + t * W + 4 * c;
            row[0] = v.x; row[1] = v.y; row[2] = v.z; row[3] = v.w;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int s = s0 + lane, pos = base + s, rpos = pos + pos_offset;
    if (s >= S || pos < 0 || pos >= T_cap || rpos < 0 || rpos >= table_len) return;
    uint16_t *vc = vt + ((size_t)b * Hkv + hk) * D * T_cap + pos;
    const int dpw = D / 4;                                 // dims per wave
    for (int d = w * dpw; d < (w + 1) * dpw; ++d) {
        const uint32_t word = tile[lane * W + (d >> 1)];
        vc[(size_t)d * T_cap] = (uint16_t)((d & 1) ? (word >> 16) : (word & 0xFFFFu));
    }
}

// ---------------------------------------------------------------- attention
//
// softmax(q k^T * scale + causal mask) v per query head, GQA heads sharing one KV
// head (attention.py:436-466).  One wave owns 16 "columns" = (position, q head)
// pairs that share a KV head, and walks the keys in blocks of 32:
//   S^T[32 keys x 16 cols] = K[keys, D] . Q^T       (2 x D/32 MFMA 16x16x32)
//   online softmax down each column (fp32, exp2 domain)
//   O^T[D x 16 cols]      += Vt[D, keys] . P^T      (D/16 MFMA 16x16x32)
// With S^T in the D layout (lane = column, 4 keys per lane-group and tile) and the
// block's keys permuted into its rows (attn_load), lane group g holds keys
// 8g .. 8g + 7 in order: exactly the k slots of operand B of the second product,
// and Vt is read for the same keys, so no LDS round trip is needed.
// The probabilities enter the second product as bf16 (as in flash attention).
// Keys may be split over waves (decode); partial (m, l, O) then go to a
// workspace and attn_combine_kernel merges them.
struct AttnArgs {
    const uint16_t *q;
    long q_stride;           // elements between token rows; head h at +h*D
    const uint16_t *kc;
    const uint16_t *vt;
    const int32_t *cache_len; // positions cached before this call's S new ones
    uint16_t *out;
    long out_stride;
    float *part;             // [B, H, S, nsplit, D + 4] when nsplit > 1: o[D], m, l, pad
    const float *mask;       // additive mask, element (b, h, s, t) at b*msb + h*msh + s*mss + t*mst
    long msb, msh, mss, mst;
    int B, S, H, Hkv, T_cap;
    int R, Rc, Pw, hgroups, npb;
    int kps, nsplit;
    float scale_log2;        // scale * log2(e)
};

constexpr int ATTN_WAVES = 4;
constexpr int ATTN_KB = 32;                       // keys per block
constexpr int ATTN_STRIDE = ATTN_WAVES * ATTN_KB;  // a workgroup's waves take interleaved blocks

// One key block's operands, loaded together: K rows for S^T (two 16-key tiles x
// D/32 k-steps) and Vt rows for O^T (D/16 tiles x keys {4g..4g+3, 16+4g..16+4g+3}).
// A block's keys are permuted on the way into S^T so that lane group g ends up with
// the 8 consecutive keys kb + 8g .. kb + 8g + 7 (tile 0 row r = key 8 (r / 4) + r % 4,
// tile 1 row r = key 8 (r / 4) + 4 + r % 4): the probabilities are then operand B of
// O^T in natural key order, and each lane's V^T operand is one 16-byte load of 8
// consecutive cached keys (a V^T row's 64 bytes of the block in one instruction's
// 4 lanes, rather than 32-byte halves in two).
template <int D>
struct AttnBlock {
    uint4 k[2][D / 32];
    uint4 v[D / 16];
};

template <int D>
__device__ __forceinline__ void attn_load(AttnBlock<D> &blk, const uint16_t *kbase, const uint16_t *vbase, int T_cap,
                                          int kb, int c, int g) {
    const int k0 = kb + 8 * (c >> 2) + (c & 3);
#pragma unroll
    for (int u = 0; u < D / 32; ++u) {
        blk.k[0][u] = *reinterpret_cast<const uint4 *>(kbase + (size_t)k0 * D + 32 * u + 8 * g);
        blk.k[1][u] = *reinterpret_cast<const uint4 *>(kbase + (size_t)(k0 + 4) * D + 32 * u + 8 * g);
    }
#pragma unroll
    for (int n = 0; n < D / 16; ++n)
        blk.v[n] = *reinterpret_cast<const uint4 *>(vbase + (size_t)(16 * n + c) * T_cap + kb + 8 * g);
}

// S^T, masked online softmax and O^T update for one block of 32 keys.  Cache slots
// at or past vend may hold anything, NaN included: in the block that reaches them
// their V pieces are zeroed, so that their zero probabilities meet no NaN.
// With MASKED, mrow[key * mst] (the column's row of the additive mask) is added to
// each score the column may see (attention.py:449-450: scores * scale + mask).
template <int D, bool MASKED = false>
__device__ __forceinline__ void attn_block(const AttnBlock<D> &blk, const bf16x8_t *qv, int kb, int limit, int vend,
                                           int g, float scale_log2, float &m, float &lsum, f4 *o,
                                           const float *mrow = nullptr, long mst = 0) {
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < D / 32; ++u) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(blk.k[0][u]), qv[u], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(blk.k[1][u]), qv[u], s1, 0, 0, 0);
    }
    // sv[j]: key kb + 8 g + j
    float sv[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        sv[r] = (kb + 8 * g + r <= limit) ? s0[r] * scale_log2 : -INFINITY;
        sv[4 + r] = (kb + 8 * g + 4 + r <= limit) ? s1[r] * scale_log2 : -INFINITY;
    }
    if (MASKED) {
        // The scores are in log2 units, so the mask is scaled by log2(e).  A finite mask
        // value stays finite: one below -FLT_MAX / log2(e) (finfo(float32).min, the
        // usual padding value) is clamped to -FLT_MAX instead of overflowing to -inf.
        // The reference adds it unscaled in fp32 and gets a finite score, so a row whose
        // visible keys all carry it gets uniform weights there, and must not become 0/0
        // here.  -inf stays -inf.
        constexpr float LOG2E = 1.4426950408889634f;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int key = kb + 8 * g + r;
            if (key <= limit) {
                const float mv = mrow[(long)key * mst];
                sv[r] += (mv == -INFINITY) ? -INFINITY : fmaxf(mv * LOG2E, -FLT_MAX);
            }
        }
    }
    float bm = sv[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) bm = fmaxf(bm, sv[r]);
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float mn = fmaxf(m, bm);
    const float alpha = (mn == -INFINITY) ? 1.f : exp2f(m - mn);
    float p[8], ps = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        p[r] = (sv[r] == -INFINITY) ? 0.f : exp2f(sv[r] - mn);
        ps += p[r];
    }
    lsum = lsum * alpha + ps;
    m = mn;
    const bf16x8_t pb8 = as_bf16x8(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                   pack_bf16x2(p[6], p[7]));
    // word i of a lane's V^T piece: keys kb + 8g + 2i, + 1
    uint32_t mk[4] = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu};
    if (kb + ATTN_KB > vend) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = kb + 8 * g + 2 * i;
            mk[i] = (k < vend ? 0xFFFFu : 0u) | (k + 1 < vend ? 0xFFFF0000u : 0u);
        }
    }
#pragma unroll
    for (int n = 0; n < D / 16; ++n) {
        f4 acc = o[n];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= alpha;
        o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(blk.v[n].x & mk[0], blk.v[n].y & mk[1], blk.v[n].z & mk[2], blk.v[n].w & mk[3]), pb8, acc,
            0, 0, 0);
    }
}

// A workgroup owns 16 columns and one key range [k_lo, k_hi); its 4 waves take the
// range's 32-key blocks round-robin (next block prefetched while one is computed),
// then merge their (m, l, O) through LDS.  With one key range the merged result is
// the output; with several it is a partial for attn_combine_kernel.
template <int D, bool MASKED>
__global__ void __launch_bounds__(64 * ATTN_WAVES) attn_kernel(AttnArgs a) {
    constexpr int U = D / 32;
    constexpr int DT = D / 16;
    __shared__ float sm_m[ATTN_WAVES][16], sm_l[ATTN_WAVES][16];
    __shared__ float sm_o[ATTN_WAVES][D][17];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    long t = blockIdx.x;
    const int sp = (int)(t % a.nsplit); t /= a.nsplit;
    const int pb = (int)(t % a.npb); t /= a.npb;
    const int hg = (int)(t % a.hgroups); t /= a.hgroups;
    const int hk = (int)(t % a.Hkv);
    const int b = (int)(t / a.Hkv);

    const int T = a.cache_len[0] + a.S;   // cached positions, the S new ones included
    const int off = T - a.S;
    const int maxpos = min(pb * a.Pw + a.Pw - 1, a.S - 1);
    const int k_lo = sp * a.kps;
    const int k_hi = min(min(k_lo + a.kps, T), maxpos + off + 1);
    if (k_lo >= T) return;   // a range wholly past the cache: the combine never reads it

    auto col_info = [&](int cc, int &pos, int &h) {
        const int hr = hg * 16 + (cc % a.Rc);
        pos = pb * a.Pw + cc / a.Rc;
        h = hk * a.R + hr;
        return (cc < a.Pw * a.Rc) && (hr < a.R) && (pos < a.S);
    };
    int pos, h;
    const bool col_ok = col_info(c, pos, h);
    const int limit = col_ok ? min(pos + off, T - 1) : -1;   // last key this column may see
    const float *mrow = MASKED && col_ok ? a.mask + b * a.msb + h * a.msh + pos * a.mss : nullptr;

    bf16x8_t qv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (col_ok)
            v = *reinterpret_cast<const uint4 *>(a.q + ((size_t)b * a.S + pos) * a.q_stride + (size_t)h * D + 32 * u + 8 * g);
        qv[u] = as_bf16x8(v);
    }
    const uint16_t *kbase = a.kc + ((size_t)b * a.Hkv + hk) * a.T_cap * D;
    const uint16_t *vbase = a.vt + ((size_t)b * a.Hkv + hk) * D * a.T_cap;

    float m = -INFINITY, lsum = 0.f;
    f4 o[DT];
#pragma unroll
    for (int n = 0; n < DT; ++n) o[n] = f4{0.f, 0.f, 0.f, 0.f};

    // Loads are unconditional (a wave past its range reloads its current block, an
    // L1/L2 hit): a load issued only on some paths makes the compiler wait for every
    // outstanding load, the prefetch included, before the current block's compute.
    AttnBlock<D> cur, nxt;
    const int clampk = a.T_cap - ATTN_KB;
    int kb = k_lo + ATTN_KB * w;
    attn_load<D>(cur, kbase, vbase, a.T_cap, min(kb, clampk), c, g);
    while (true) {
        const int kn = kb + ATTN_STRIDE;
        attn_load<D>(nxt, kbase, vbase, a.T_cap, min(kn < k_hi ? kn : kb, clampk), c, g);
        if (kb < k_hi) attn_block<D, MASKED>(cur, qv, kb, limit, T, g, a.scale_log2, m, lsum, o, mrow, a.mst);
        if (kn >= k_hi) break;
        const int kn2 = kn + ATTN_STRIDE;
        attn_load<D>(cur, kbase, vbase, a.T_cap, min(kn2 < k_hi ? kn2 : kn, clampk), c, g);
        attn_block<D, MASKED>(nxt, qv, kn, limit, T, g, a.scale_log2, m, lsum, o, mrow, a.mst);
        if (kn2 >= k_hi) break;
        kb = kn2;
    }
    float ltot = lsum + __shfl_xor(lsum, 16);
    ltot += __shfl_xor(ltot, 32);

    // ---- merge the 4 waves: o[n][r] is O^T[dim 16n + 4g + r][column c]
    if (g == 0) {
        sm_m[w][c] = m;
        sm_l[w][c] = ltot;
    }
#pragma unroll
    for (int n = 0; n < DT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) sm_o[w][16 * n + 4 * g + r][c] = o[n][r];
    __syncthreads();
    const int cc = threadIdx.x & 15;
    int cpos, ch;
    if (!col_info(cc, cpos, ch)) return;
    float M = sm_m[0][cc];
#pragma unroll
    for (int i = 1; i < ATTN_WAVES; ++i) M = fmaxf(M, sm_m[i][cc]);
    float wt[ATTN_WAVES], L = 0.f;
#pragma unroll
    for (int i = 0; i < ATTN_WAVES; ++i) {
        wt[i] = (sm_m[i][cc] == -INFINITY) ? 0.f : exp2f(sm_m[i][cc] - M);
        L += wt[i] * sm_l[i][cc];
    }
    constexpr int PER = D * 16 / (64 * ATTN_WAVES);      // dims per thread
    const int d0 = threadIdx.x >> 4;                     // 0..15
    if (a.nsplit == 1) {
        const float inv = 1.f / L;
        uint16_t *orow = a.out + ((size_t)b * a.S + cpos) * a.out_stride + (size_t)ch * D;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int d = d0 + 16 * j;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < ATTN_WAVES; ++i) acc += wt[i] * sm_o[i][d][cc];
            orow[d] = (uint16_t)f2bf(acc * inv);
        }
    } else {
        float *pp = a.part + ((((size_t)b * a.H + ch) * a.S + cpos) * a.nsplit + sp) * (D + 4);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int d = d0 + 16 * j;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < ATTN_WAVES; ++i) acc += wt[i] * sm_o[i][d][cc];
            pp[d] = acc;
        }
        if (d0 == 0) {
            pp[D] = M;
            pp[D + 1] = L;
        }
    }
}

// Merges the key-range partials of one (b, h, position) per wave: lane i holds
// partial i's (m, l); each lane then sums dims lane, lane + 64 over the partials.
template <int D>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a) {
    const long wid = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (wid >= (long)a.B * a.H * a.S) return;
    const int T = a.cache_len[0] + a.S;
    const int used = min(a.nsplit, (T + a.kps - 1) / a.kps);   // <= 64 by construction
    const float *pp = a.part + wid * a.nsplit * (D + 4);
    constexpr int PER = D / 64;
    // the first PF partials' values are loaded with the (m, l) pairs, in one round trip
    // (past `used` they repeat the last stored partial and are not added)
    constexpr int PF = 8;
    float vf[PF][PER];
#pragma unroll
    for (int k = 0; k < PF; ++k)
#pragma unroll
        for (int e = 0; e < PER; ++e) vf[k][e] = pp[(size_t)min(k, used - 1) * (D + 4) + lane + 64 * e];
    const float mi = lane < used ? pp[(size_t)lane * (D + 4) + D] : -INFINITY;
    const float li = lane < used ? pp[(size_t)lane * (D + 4) + D + 1] : 0.f;
    float M = mi;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    const float wi = (mi == -INFINITY) ? 0.f : exp2f(mi - M);
    const float L = wave_sum(wi * li);
    float acc[PER] = {};
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        const float wk = __shfl(wi, k);
        if (k < used) {
#pragma unroll
            for (int e = 0; e < PER; ++e) acc[e] += wk * vf[k][e];
        }
    }
    int i = PF;
    for (; i + 4 <= used; i += 4) {
        float v[4][PER];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < PER; ++e) v[k][e] = pp[(size_t)(i + k) * (D + 4) + lane + 64 * e];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float wk = __shfl(wi, i + k);
#pragma unroll
            for (int e = 0; e < PER; ++e) acc[e] += wk * v[k][e];
        }
    }
    for (; i < used; ++i) {
        const float wk = __shfl(wi, i);
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[e] += wk * pp[(size_t)i * (D + 4) + lane + 64 * e];
    }
    const int bh = (int)(wid / a.S), pos = (int)(wid % a.S);
    const int b = bh / a.H, h = bh % a.H;
    uint16_t *orow = a.out + ((size_t)b * a.S + pos) * a.out_stride + (size_t)h * D;
    const float inv = 1.f / L;
#pragma unroll
    for (int e = 0; e < PER; ++e) orow[lane + 64 * e] = (uint16_t)f2bf(acc[e] * inv);
}

// ---------------------------------------------------------------- decode attention
//
// One new position per sequence (S = 1, the decode step): RoPE of q and of the new
// k, the cache append and attention over the cached keys plus the new one, in one
// launch (attention.py:421-466 for one token).  Workgroup (key range sp, kv head
// hk, sequence b), 4 waves:
// * the first cached-key block's loads are issued before anything else; then q of
//   the R query heads sharing the kv head is read from the q|k|v row and rotated on
//   the way in, with rope_append_kernel's arithmetic;
// * the cached keys [k_lo, min(k_lo + kps, T - 1)) go through attn_block as in
//   attn_kernel;
// * the new key and value (position T - 1) never make a round trip through memory
//   inside the kernel: the range holding T - 1 adds them to wave 0's softmax state
//   from registers, and writes them into the cache for later steps;
// * the waves merge in LDS; with one range the result is the output, otherwise the
//   range's partial goes to the workspace in attn_kernel's layout and
//   attn_combine_kernel merges the ranges (a cross-XCD merge inside the kernel
//   costs more than the second launch: coherent stores, a device-scope count and
//   coherent loads are each a trip to memory).
struct AttnDecArgs {
    const uint16_t *qkv;
    long qkv_stride;         // elements between sequences' rows: q heads, then k, then v
    const float *cos_t;      // [table_len, D / 2]
    const float *sin_t;
    int table_len, pos_offset;
    uint16_t *kc;            // [B, Hkv, T_cap, D]
    uint16_t *vt;            // [B, Hkv, D, T_cap]
    int T_cap;
    const int32_t *cache_len; // cached positions before this token = its slot
    uint16_t *out;
    long out_stride;
    float *part;             // [B, H, 1, nsplit, D + 4] when nsplit > 1: O[D], m, l, pad
    int H, Hkv, R, kps, nsplit;
    float scale_log2;
    const float *mask;       // attn_decode_kernel<D, true>: additive mask, element (b, h, 0, t) at
    long msb, msh, mst;      // mask + b msb + h msh + t mst
};

// dims [i0, i0 + 8) of the first half of a head and their partners i0 + D/2,
// rotated with the table values (cv, sv) of those dims:
// bf16(x1 c - x2 s), bf16(x2 c + x1 s)
__device__ __forceinline__ void rope_pair8(uint4 lo, uint4 hi, const float *cv, const float *sv, uint4 &olo,
                                           uint4 &ohi) {
    uint32_t a[4], bb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float r1[2], r2[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = 2 * e + k;
            const float x1 = bfe(lo, i), x2 = bfe(hi, i);
            r1[k] = add_rn(mul_rn(x1, cv[i]), mul_rn(-x2, sv[i]));
            r2[k] = add_rn(mul_rn(x2, cv[i]), mul_rn(x1, sv[i]));
        }
        a[e] = pack_bf16x2(r1[0], r1[1]);
        bb[e] = pack_bf16x2(r2[0], r2[1]);
    }
    olo = make_uint4(a[0], a[1], a[2], a[3]);
    ohi = make_uint4(bb[0], bb[1], bb[2], bb[3]);
}

// MASKED: the additive mask of the new position's row (attention.py:449-450), added to
// every visible score, the new key's included, as attn_kernel<D, true> adds it.
template <int D, bool MASKED>
__global__ void __launch_bounds__(64 * ATTN_WAVES) attn_decode_kernel(AttnDecArgs a) {
    constexpr int U = D / 32;
    constexpr int DT = D / 16;
    constexpr int HALF = D / 2;
    __shared__ float sm_m[ATTN_WAVES][16], sm_l[ATTN_WAVES][16];
    __shared__ float sm_o[ATTN_WAVES][D][17];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int sp = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
    const int bh = b * a.Hkv + hk;

    // Loads that do not depend on the cache length go out first, in the order they
    // are needed (vmcnt retires in order): q, the range's first key block, then
    // (after the length arrives) the table row and the new key and value.
    // (Unconditional loads: columns past R read head R - 1 and are masked later; a
    // conditional load would make the compiler wait for it on the spot.  The length
    // is read first, as a scalar load that is waited for only where it is used.)
    const int pos = a.cache_len[0];                 // slot of the new position
    const uint16_t *row = a.qkv + (size_t)b * a.qkv_stride;
    const bool col_ok = c < a.R;
    const float *mrow = MASKED && col_ok ? a.mask + b * a.msb + (long)(hk * a.R + c) * a.msh : nullptr;
    uint4 qraw[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        qraw[u] = *reinterpret_cast<const uint4 *>(row + (size_t)(hk * a.R + min(c, a.R - 1)) * D + 32 * u + 8 * g);
    const int k_lo = sp * a.kps;
    const uint16_t *kbase = a.kc + (size_t)bh * a.T_cap * D;
    const uint16_t *vbase = a.vt + (size_t)bh * D * a.T_cap;
    AttnBlock<D> cur, nxt;
    const int clampk = a.T_cap - ATTN_KB;
    int kb = k_lo + ATTN_KB * w;
    attn_load<D>(cur, kbase, vbase, a.T_cap, min(kb, clampk), c, g);
    asm volatile("" ::: "memory");                  // keep these loads ahead of the length check below

    const int rpos = pos + a.pos_offset;            // its rotary position
    // the host sizes cache and tables for every launch; a counter that has run past
    // them (a stale replay) leaves everything untouched instead of reading or
    // writing out of bounds
    if (pos < 0 || pos >= a.T_cap || rpos < 0 || rpos >= a.table_len) return;
    const int T = pos + 1;                          // keys after the append
    if (k_lo >= T) return;                          // a range wholly past the keys: the combine never reads it
    const int k_hi = min(k_lo + a.kps, T - 1);      // cached keys of this range
    const bool has_new = T - 1 < k_lo + a.kps;      // the range holding the new position
    const bool add_new = has_new && w == 0;         // its wave 0 folds the new key in
    const int limit = col_ok ? T - 2 : -1;          // last cached key a column may see (all of them)

    const float *ct = a.cos_t + (size_t)rpos * HALF, *st = a.sin_t + (size_t)rpos * HALF;
    float cv[U / 2][8], sv[U / 2][8];
#pragma unroll
    for (int u = 0; u < U / 2; ++u) {
        const float4 c0 = *reinterpret_cast<const float4 *>(ct + 32 * u + 8 * g);
        const float4 c1 = *reinterpret_cast<const float4 *>(ct + 32 * u + 8 * g + 4);
        const float4 s0 = *reinterpret_cast<const float4 *>(st + 32 * u + 8 * g);
        const float4 s1 = *reinterpret_cast<const float4 *>(st + 32 * u + 8 * g + 4);
        cv[u][0] = c0.x; cv[u][1] = c0.y; cv[u][2] = c0.z; cv[u][3] = c0.w;
        cv[u][4] = c1.x; cv[u][5] = c1.y; cv[u][6] = c1.z; cv[u][7] = c1.w;
        sv[u][0] = s0.x; sv[u][1] = s0.y; sv[u][2] = s0.z; sv[u][3] = s0.w;
        sv[u][4] = s1.x; sv[u][5] = s1.y; sv[u][6] = s1.z; sv[u][7] = s1.w;
    }
    uint4 knew[U];                                  // (loaded by every wave: see above)
    uint2 vnew[DT];
    {
        const uint16_t *krow = row + (size_t)(a.H + hk) * D;
        const uint16_t *vrow = row + (size_t)(a.H + a.Hkv + hk) * D;
#pragma unroll
        for (int u = 0; u < U; ++u) knew[u] = *reinterpret_cast<const uint4 *>(krow + 32 * u + 8 * g);
#pragma unroll
        for (int n = 0; n < DT; ++n) vnew[n] = *reinterpret_cast<const uint2 *>(vrow + 16 * n + 4 * g);
    }
    bf16x8_t qv[U];
#pragma unroll
    for (int u = 0; u < U / 2; ++u) {
        uint4 lo, hi;
        rope_pair8(qraw[u], qraw[u + U / 2], cv[u], sv[u], lo, hi);
        qv[u] = as_bf16x8(lo);
        qv[u + U / 2] = as_bf16x8(hi);
    }

    float m = -INFINITY, lsum = 0.f;
    f4 o[DT];
#pragma unroll
    for (int n = 0; n < DT; ++n) o[n] = f4{0.f, 0.f, 0.f, 0.f};

    // cached keys.  One block per wave (the usual decode split) needs no prefetch: a
    // useless one would also hold vmcnt slots that the append's stores then wait for.
    if (kb + ATTN_STRIDE >= k_hi) {
        if (kb < k_hi) attn_block<D, MASKED>(cur, qv, kb, limit, T - 1, g, a.scale_log2, m, lsum, o, mrow, a.mst);
    } else {
        // the loop of attn_kernel (unconditional, clamped loads)
        while (true) {
            const int kn = kb + ATTN_STRIDE;
            attn_load<D>(nxt, kbase, vbase, a.T_cap, min(kn < k_hi ? kn : kb, clampk), c, g);
            if (kb < k_hi) attn_block<D, MASKED>(cur, qv, kb, limit, T - 1, g, a.scale_log2, m, lsum, o, mrow, a.mst);
            if (kn >= k_hi) break;
            const int kn2 = kn + ATTN_STRIDE;
            attn_load<D>(cur, kbase, vbase, a.T_cap, min(kn2 < k_hi ? kn2 : kn, clampk), c, g);
            attn_block<D, MASKED>(nxt, qv, kn, limit, T - 1, g, a.scale_log2, m, lsum, o, mrow, a.mst);
            if (kn2 >= k_hi) break;
            kb = kn2;
        }
    }

    // the new key and value: rotate k, append k and v, fold them into wave 0's state
    if (add_new) {
        uint4 kr[U];
#pragma unroll
        for (int u = 0; u < U / 2; ++u) rope_pair8(knew[u], knew[u + U / 2], cv[u], sv[u], kr[u], kr[u + U / 2]);
        // append, one dim (pair) per lane: k dims i and i + D/2, v dims d (the
        // rotation repeated in this layout, same arithmetic)
        {
            const uint16_t *krow = row + (size_t)(a.H + hk) * D;
            const uint16_t *vrow = row + (size_t)(a.H + a.Hkv + hk) * D;
            uint16_t *kdst = a.kc + ((size_t)bh * a.T_cap + pos) * D;
            uint16_t *vdst = a.vt + (size_t)bh * D * a.T_cap + pos;
            for (int i = lane; i < HALF; i += 64) {
                const float x1 = bf2f(krow[i]), x2 = bf2f(krow[i + HALF]);
                kdst[i] = (uint16_t)f2bf(add_rn(mul_rn(x1, ct[i]), mul_rn(-x2, st[i])));
                kdst[i + HALF] = (uint16_t)f2bf(add_rn(mul_rn(x2, ct[i]), mul_rn(x1, st[i])));
            }
            for (int d = lane; d < D; d += 64) vdst[(size_t)d * a.T_cap] = vrow[d];
        }
        // score of the new key for column c: the lane's 8 dims per u, then across g
        float dot = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) dot = fmaf(bfe(__builtin_bit_cast(uint4, qv[u]), e), bfe(kr[u], e), dot);
        dot += __shfl_xor(dot, 16);
        dot += __shfl_xor(dot, 32);
        float sn = col_ok ? dot * a.scale_log2 : -INFINITY;
        if (MASKED && col_ok) {
            // attn_block's scaling and clamp of the mask value
            const float mv = mrow[(long)(T - 1) * a.mst];
            sn += (mv == -INFINITY) ? -INFINITY : fmaxf(mv * 1.4426950408889634f, -FLT_MAX);
        }
        const float mn = fmaxf(m, sn);
        const float alpha = (mn == -INFINITY) ? 1.f : exp2f(m - mn);
        const float p = (sn == -INFINITY) ? 0.f : exp2f(sn - mn);
        lsum = lsum * alpha + (g == 0 ? p : 0.f);
        m = mn;
        const float pb = bf2f(f2bf(p));             // probabilities enter the PV product as bf16
#pragma unroll
        for (int n = 0; n < DT; ++n) {
            const float v4[4] = {__uint_as_float(vnew[n].x << 16), __uint_as_float(vnew[n].x & 0xFFFF0000u),
                                 __uint_as_float(vnew[n].y << 16), __uint_as_float(vnew[n].y & 0xFFFF0000u)};
#pragma unroll
            for (int r = 0; r < 4; ++r) o[n][r] = fmaf(pb, v4[r], o[n][r] * alpha);
        }
    }
    float ltot = lsum + __shfl_xor(lsum, 16);
    ltot += __shfl_xor(ltot, 32);

    // ---- merge the 4 waves (as attn_kernel): o[n][r] is O^T[dim 16n + 4g + r][column c]
    if (g == 0) {
        sm_m[w][c] = m;
        sm_l[w][c] = ltot;
    }
#pragma unroll
    for (int n = 0; n < DT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) sm_o[w][16 * n + 4 * g + r][c] = o[n][r];
    __syncthreads();
    const int cc = threadIdx.x & 15;
    if (cc >= a.R) return;
    float M = sm_m[0][cc];
#pragma unroll
    for (int i = 1; i < ATTN_WAVES; ++i) M = fmaxf(M, sm_m[i][cc]);
    float wt[ATTN_WAVES], L = 0.f;
#pragma unroll
    for (int i = 0; i < ATTN_WAVES; ++i) {
        wt[i] = (sm_m[i][cc] == -INFINITY) ? 0.f : exp2f(sm_m[i][cc] - M);
        L += wt[i] * sm_l[i][cc];
    }
    constexpr int PER = D * 16 / (64 * ATTN_WAVES);      // dims per thread
    const int d0 = threadIdx.x >> 4;                     // 0..15
    const int h = hk * a.R + cc;
    if (a.nsplit == 1) {
        const float inv = 1.f / L;
        uint16_t *orow = a.out + (size_t)b * a.out_stride + (size_t)h * D;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int d = d0 + 16 * j;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < ATTN_WAVES; ++i) acc += wt[i] * sm_o[i][d][cc];
            orow[d] = (uint16_t)f2bf(acc * inv);
        }
    } else {
        float *pp = a.part + (((size_t)b * a.H + h) * a.nsplit + sp) * (D + 4);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int d = d0 + 16 * j;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < ATTN_WAVES; ++i) acc += wt[i] * sm_o[i][d][cc];
            pp[d] = acc;
        }
        if (d0 == 0) {
            pp[D] = M;
            pp[D + 1] = L;
        }
    }
}

// ---------------------------------------------------------------- SiLU gate
//
// out = (g / (1 + exp(-g))) * u for the fused [rows, 2I] gate|up product
// (parallel/mlp.py:161-162, 241-245).
__global__ void __launch_bounds__(256)
silu_mul_kernel(const uint16_t *__restrict__ gu, uint16_t *__restrict__ out, long rows, int I) {
    const long nv = rows * (I >> 3);
    const int vpr = I >> 3;
    for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < nv; idx += (long)gridDim.x * blockDim.x) {
        const long r = idx / vpr;
        const int v = (int)(idx - r * vpr);
        const uint4 gv = reinterpret_cast<const uint4 *>(gu + (size_t)r * 2 * I)[v];
        const uint4 uv = reinterpret_cast<const uint4 *>(gu + (size_t)r * 2 * I + I)[v];
        reinterpret_cast<uint4 *>(out + (size_t)r * I)[v] = silu_mul_bf16x8(gv, uv);
    }
}

// ---------------------------------------------------------------- greedy argmax
//
// First index of the maximum of each row (worker/executor.py:276-278 at
// temperature 0, numpy/MLX argmax semantics): NaN counts as the maximum and
// -0.0 equals +0.0.  Keys (argmax_key: order-preserving 16-bit image, ~index)
// packed in 64 bits so one max-reduction yields the largest value at the smallest
// index.
__global__ void __launch_bounds__(1024)
argmax_kernel(const uint16_t *__restrict__ logits, long V, int32_t *__restrict__ ids,
              int32_t *__restrict__ tokens, long tok_stride, long tok_cols, const int32_t *__restrict__ step) {
    const int row = blockIdx.x;
    const uint16_t *lr = logits + (size_t)row * V;
    unsigned long long best = 0;
    // vector path: 16-byte rows, and the in-thread sequence number (below 8 per
    // uint4 times the uint4s per thread) fits 16 bits
    const bool vec = ((V & 7) == 0) && (V / 8 + blockDim.x - 1) / blockDim.x <= 8192;
    if (vec) {
        // 16 loads per thread in flight before any is reduced; within the thread a
        // 32-bit key (order-preserving value << 16 | 0xFFFF - s, s = the element's
        // sequence number in this thread, increasing with its index) so each element
        // costs one max; the winner is widened to the 64-bit (value, index) key below
        constexpr int U = 16;
        const uint4 *lv = reinterpret_cast<const uint4 *>(lr);
        const long n8 = V / 8;
        uint32_t bl = 0u;                                   // 0: no element (no real key is 0)
        int seq = 0;
        for (long i0 = threadIdx.x; i0 < n8; i0 += (long)U * blockDim.x) {
            uint4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long i = i0 + (long)u * blockDim.x;
                v[u] = i < n8 ? lv[i] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long i = i0 + (long)u * blockDim.x;
                if (i < n8) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t w = e < 2 ? v[u].x : e < 4 ? v[u].y : e < 6 ? v[u].z : v[u].w;
                        const uint32_t key = (uint32_t)(argmax_key((e & 1) ? (w >> 16) : w, 0u) >> 32);
                        const uint32_t kk = (key << 16) | (0xFFFFu - (uint32_t)(seq + 8 * u + e));
                        bl = kk > bl ? kk : bl;
                    }
                }
            }
            seq += 8 * U;
        }
        if (bl != 0u) {
            const uint32_t sq = 0xFFFFu - (bl & 0xFFFFu);
            const uint32_t idx = 8u * ((uint32_t)threadIdx.x + (sq >> 3) * blockDim.x) + (sq & 7u);
            best = ((unsigned long long)(bl >> 16) << 32) | (0xFFFFFFFFu - idx);
        }
    } else {
        for (long i = threadIdx.x; i < V; i += blockDim.x) {
            const unsigned long long kk = argmax_key(lr[i], (uint32_t)i);
            best = kk > best ? kk : best;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o);
        best = other > best ? other : best;
    }
    __shared__ unsigned long long red[16];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i) best = red[i] > best ? red[i] : best;
        const int32_t id = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
        ids[row] = id;
        const long col = step ? step[0] : 0;
        if (tokens && col >= 0 && col < tok_cols) tokens[(size_t)row * tok_stride + col] = id;
    }
}

// out = bf16(a + b) elementwise (the residual adds of transformer.py:246, 252 where
// no normalisation follows).
__global__ void __launch_bounds__(256)
add_bf16_kernel(const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, uint16_t *__restrict__ out, long nv) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += (long)gridDim.x * blockDim.x)
        reinterpret_cast<uint4 *>(out)[i] = add_bf16x8(reinterpret_cast<const uint4 *>(a)[i], reinterpret_cast<const uint4 *>(b)[i]);
}

__global__ void add_i32_kernel(int32_t *p, int n, int32_t delta) {
    const int i = threadIdx.x;
    if (i < n) p[i] += delta;
}

// ---------------------------------------------------------------- host side

namespace {

struct AttnPlan {
    AttnArgs a;
    long blocks;
};

void plan_attention(long B, long S, long H, long Hkv, long D, long T_cap, AttnPlan *pl) {
    AttnArgs &a = pl->a;
    a = AttnArgs{};
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.Hkv = (int)Hkv; a.T_cap = (int)T_cap;
    a.R = (int)(H / Hkv);
    a.Rc = a.R < 16 ? a.R : 16;
    a.Pw = 16 / a.Rc;
    a.hgroups = (a.R + 15) / 16;
    a.npb = (int)((S + a.Pw - 1) / a.Pw);
    const long base = B * Hkv * a.hgroups * a.npb;
    // split the keys into ranges when the (batch, head, position) workgroups alone
    // cannot fill the GPU; a range covers one block per wave at least, and at most
    // 64 ranges are merged (one per lane of the combine).  The attention kernels take
    // all 256 VGPRs, so one 4-wave workgroup runs per CU: the target is one round of
    // workgroups (two rounds of half-length ranges measured 20-28 % slower at batch
    // 4-32 decode)
    const long target = device_info().num_cus;
    int nsplit = 1;
    if (base < target && T_cap > ATTN_STRIDE) {
        long want = (target + base - 1) / base;
        long kps = (T_cap + want - 1) / want;
        kps = ((kps + ATTN_STRIDE - 1) / ATTN_STRIDE) * ATTN_STRIDE;
        long cap64 = ((T_cap + 63) / 64 + ATTN_STRIDE - 1) / ATTN_STRIDE * ATTN_STRIDE;
        if (kps < cap64) kps = cap64;
        nsplit = (int)((T_cap + kps - 1) / kps);
        a.kps = (int)kps;
    }
    if (nsplit <= 1) {
        nsplit = 1;
        a.kps = (int)T_cap;
    }
    a.nsplit = nsplit;
    pl->blocks = base * nsplit;
}

}  // namespace

int launch_rms_norm(const uint16_t *x, const uint16_t *res, const uint16_t *w, uint16_t *y, uint16_t *h_out,
                    long rows, long D, float eps, hipStream_t stream) {
    if (!x || !w || !y) return set_error(SC_EINVAL, "rms_norm: null pointer");
    if (rows < 0 || D <= 0 || D % 8 || D > (long)NORM_THREADS * NORM_MAXV * 8)
        return set_error(SC_EINVAL, "rms_norm: D=%ld must be a positive multiple of 8 up to %d", D,
                         NORM_THREADS * NORM_MAXV * 8);
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)y | (uintptr_t)res | (uintptr_t)h_out) % 16)
        return set_error(SC_EINVAL, "rms_norm: pointers must be 16-byte aligned");
    if (rows == 0) return SC_OK;
    hipLaunchKernelGGL(add_rms_norm_kernel, dim3((unsigned)rows), dim3(NORM_THREADS), 0, stream, x, res, w, y,
                       h_out, (int)D, eps);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_split_add_rms_norm(const float *partials, int splits, const uint16_t *y_in, const uint16_t *bias,
                              const uint16_t *res, const uint16_t *w, uint16_t *h_out, uint16_t *out, long rows, long D,
                              float eps, hipStream_t stream) {
    if ((splits > 0 ? !partials : !y_in) || !res || !w || !h_out || !out)
        return set_error(SC_EINVAL, "add_rms_norm: null pointer");
    if (rows < 0 || D <= 0 || D % 8 || D > (long)NORM_THREADS * NORM_MAXV * 8)
        return set_error(SC_EINVAL, "add_rms_norm: D=%ld must be a positive multiple of 8 up to %d", D,
                         NORM_THREADS * NORM_MAXV * 8);
    if (((uintptr_t)partials | (uintptr_t)y_in | (uintptr_t)res | (uintptr_t)w | (uintptr_t)h_out |
         (uintptr_t)out | (uintptr_t)bias) % 16)
        return set_error(SC_EINVAL, "add_rms_norm: pointers must be 16-byte aligned");
    if (rows == 0) return SC_OK;
    if (rows > 0x7FFFFFFFL) return set_error(SC_EINVAL, "add_rms_norm: too many rows");
    const int nv = (int)(D / 8);
    const int threads = nv >= PNORM_THREADS ? PNORM_THREADS : nv <= NORM_THREADS ? NORM_THREADS : (nv + 63) / 64 * 64;
    hipLaunchKernelGGL(split_add_rms_norm_kernel, dim3((unsigned)rows), dim3(threads), 0, stream, partials,
                       splits, y_in, bias, res, w, h_out, out, rows, (int)D, eps);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_rope_append(uint16_t *qkv, long qkv_stride, long B, long S, long H, long Hkv, long D,
                       const float *cos_t, const float *sin_t, long table_len, uint16_t *kc, uint16_t *vt,
                       long T_cap, const int32_t *cache_len, long pos_offset, hipStream_t stream) {
    if (!qkv || !cos_t || !sin_t || !kc || !vt || !cache_len) return set_error(SC_EINVAL, "rope_append: null pointer");
    if (B <= 0 || S <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || D <= 0 || D % 2)
        return set_error(SC_EINVAL, "rope_append: bad shape B=%ld S=%ld H=%ld Hkv=%ld D=%ld", B, S, H, Hkv, D);
    if (qkv_stride < (H + 2 * Hkv) * D) return set_error(SC_EINVAL, "rope_append: qkv_stride too small");
    if (T_cap <= 0 || table_len <= 0 || pos_offset < 0 || T_cap > 0x7FFFFFFFL || table_len > 0x7FFFFFFFL ||
        pos_offset > 0x7FFFFFFFL)
        return set_error(SC_EINVAL, "rope_append: bad capacity/table/offset");
    // many positions: v through v_append_kernel (64 tokens a workgroup), when its
    // 16-byte row loads are aligned
    const bool tiled_v = S >= 16 && D % 8 == 0 && D <= 128 && qkv_stride % 8 == 0 && (uintptr_t)qkv % 16 == 0;
    const int v_heads = tiled_v ? 0 : (int)Hkv;
    hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)(B * S), (unsigned)((H + Hkv + v_heads + 3) / 4)), dim3(256),
                       0, stream, qkv, qkv_stride, (int)S,
                       (int)H, (int)Hkv, (int)D, cos_t, sin_t, kc, vt, (int)T_cap, cache_len, (int)pos_offset,
                       (int)table_len, v_heads);
    SC_HIP_CHECK(hipGetLastError());
    if (tiled_v) {
        hipLaunchKernelGGL(v_append_kernel, dim3((unsigned)((S + VAPP_TOK - 1) / VAPP_TOK), (unsigned)Hkv, (unsigned)B),
                           dim3(256), 0, stream, qkv, qkv_stride, (int)S, (int)H, (int)Hkv, (int)D, vt, (int)T_cap,
                           cache_len, (int)pos_offset, (int)table_len);
        SC_HIP_CHECK(hipGetLastError());
    }
    return SC_OK;
}

long attention_workspace_bytes(long B, long S, long H, long Hkv, long D, long T_cap) {
    if (B <= 0 || S <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || T_cap <= 0) return 0;
    AttnPlan pl;
    plan_attention(B, S, H, Hkv, D, T_cap, &pl);
    if (pl.a.nsplit == 1) return 0;
    return B * H * S * (long)pl.a.nsplit * (D + 4) * (long)sizeof(float);
}

long attention_decode_workspace_bytes(long B, long H, long Hkv, long D, long T_cap) {
    return attention_workspace_bytes(B, 1, H, Hkv, D, T_cap);
}

// mask / ms (optional): the additive mask and its (b, h, s, t) strides, as for
// launch_attention (the s stride is unused: one position per sequence)
int launch_attention_decode(const uint16_t *qkv, long qkv_stride, long B, long H, long Hkv, long D,
                            const float *cos_t, const float *sin_t, long table_len, uint16_t *kc, uint16_t *vt,
                            long T_cap, const int32_t *cache_len, long pos_offset, float scale, uint16_t *out,
                            long out_stride, void *workspace, long workspace_bytes, hipStream_t stream,
                            const float *mask, const long *ms) {
    if (mask && (!ms || ms[0] < 0 || ms[1] < 0 || ms[2] < 0 || ms[3] < 0))
        return set_error(SC_EINVAL, "attention_decode: mask strides must be given and non-negative");
    if (!qkv || !cos_t || !sin_t || !kc || !vt || !cache_len || !out)
        return set_error(SC_EINVAL, "attention_decode: null pointer");
    if (D != 64 && D != 128) return set_error(SC_EUNSUPPORTED, "attention_decode: head_dim %ld (64 or 128 supported)", D);
    if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || H / Hkv > 16)
        return set_error(SC_EINVAL, "attention_decode: bad shape B=%ld H=%ld Hkv=%ld (at most 16 q heads per kv head)",
                         B, H, Hkv);
    if (B > 65535 || Hkv > 65535) return set_error(SC_EINVAL, "attention_decode: B and Hkv must be below 65536");
    if (T_cap <= 0 || T_cap % 32 || T_cap >= (1L << 30))
        return set_error(SC_EINVAL, "attention_decode: cache capacity %ld must be a positive multiple of 32", T_cap);
    if (table_len <= 0 || table_len >= (1L << 30) || pos_offset < 0 || pos_offset >= (1L << 30))
        return set_error(SC_EINVAL, "attention_decode: bad rotary table length or offset");
    if (qkv_stride < (H + 2 * Hkv) * D || out_stride < H * D || qkv_stride % 8 || out_stride % 4)
        return set_error(SC_EINVAL, "attention_decode: bad row strides");
    if (((uintptr_t)qkv | (uintptr_t)kc | (uintptr_t)cos_t | (uintptr_t)sin_t) % 16 || ((uintptr_t)vt | (uintptr_t)out) % 8)
        return set_error(SC_EINVAL, "attention_decode: misaligned pointers");
    AttnPlan pl;
    plan_attention(B, 1, H, Hkv, D, T_cap, &pl);
    AttnArgs ca = pl.a;                                  // the combine's view of the same plan
    ca.q = nullptr; ca.q_stride = 0; ca.kc = kc; ca.vt = vt; ca.cache_len = cache_len;
    ca.out = out; ca.out_stride = out_stride;
    ca.scale_log2 = scale * 1.4426950408889634f;
    ca.part = nullptr;
    if (ca.nsplit > 1) {
        const long need = attention_workspace_bytes(B, 1, H, Hkv, D, T_cap);
        if (!workspace || workspace_bytes < need)
            return set_error(SC_EINVAL, "attention_decode: workspace of %ld bytes required", need);
        if ((uintptr_t)workspace % 16) return set_error(SC_EINVAL, "attention_decode: workspace must be 16-byte aligned");
        ca.part = static_cast<float *>(workspace);
    }
    AttnDecArgs a;
    a.qkv = qkv; a.qkv_stride = qkv_stride;
    a.cos_t = cos_t; a.sin_t = sin_t; a.table_len = (int)table_len; a.pos_offset = (int)pos_offset;
    a.kc = kc; a.vt = vt; a.T_cap = (int)T_cap; a.cache_len = cache_len;
    a.out = out; a.out_stride = out_stride;
    a.part = ca.part;
    a.H = (int)H; a.Hkv = (int)Hkv; a.R = (int)(H / Hkv);
    a.kps = ca.kps; a.nsplit = ca.nsplit;
    a.scale_log2 = ca.scale_log2;
    const dim3 grid((unsigned)a.nsplit, (unsigned)Hkv, (unsigned)B);
    a.mask = mask;
    a.msb = mask ? ms[0] : 0; a.msh = mask ? ms[1] : 0; a.mst = mask ? ms[3] : 0;
    if (mask) {
        if (D == 128) hipLaunchKernelGGL((attn_decode_kernel<128, true>), grid, dim3(64 * ATTN_WAVES), 0, stream, a);
        else hipLaunchKernelGGL((attn_decode_kernel<64, true>), grid, dim3(64 * ATTN_WAVES), 0, stream, a);
    } else {
        if (D == 128) hipLaunchKernelGGL((attn_decode_kernel<128, false>), grid, dim3(64 * ATTN_WAVES), 0, stream, a);
        else hipLaunchKernelGGL((attn_decode_kernel<64, false>), grid, dim3(64 * ATTN_WAVES), 0, stream, a);
    }
    SC_HIP_CHECK(hipGetLastError());
    if (ca.nsplit > 1) {
        const unsigned cb = (unsigned)((B * H + 3) / 4);
        if (D == 128) hipLaunchKernelGGL(attn_combine_kernel<128>, dim3(cb), dim3(256), 0, stream, ca);
        else hipLaunchKernelGGL(attn_combine_kernel<64>, dim3(cb), dim3(256), 0, stream, ca);
        SC_HIP_CHECK(hipGetLastError());
    }
    return SC_OK;
}

// attn_prefill.hip
int launch_attn_prefill(const uint16_t *q, long q_stride, const uint16_t *kc, const uint16_t *vt, long T_cap,
                        const int32_t *cache_len, uint16_t *out, long out_stride, long B, long S, long H, long Hkv,
                        long D, float scale, hipStream_t stream, const float *mask, const long *ms);

// mask (optional): the additive mask of sc_attention_masked_bf16, element (b, h, s, t)
// at mask + b*ms[0] + h*ms[1] + s*ms[2] + t*ms[3].
int launch_attention(const uint16_t *q, long q_stride, const uint16_t *kc, const uint16_t *vt, long T_cap,
                     const int32_t *cache_len, uint16_t *out, long out_stride, long B, long S, long H, long Hkv,
                     long D, float scale, void *workspace, long workspace_bytes, hipStream_t stream,
                     const float *mask, const long *ms) {
    if (!q || !kc || !vt || !cache_len || !out) return set_error(SC_EINVAL, "attention: null pointer");
    if (D != 64 && D != 128) return set_error(SC_EUNSUPPORTED, "attention: head_dim %ld (64 or 128 supported)", D);
    if (B <= 0 || S <= 0 || H <= 0 || Hkv <= 0 || H % Hkv)
        return set_error(SC_EINVAL, "attention: bad shape B=%ld S=%ld H=%ld Hkv=%ld", B, S, H, Hkv);
    if (T_cap <= 0 || T_cap % 32) return set_error(SC_EINVAL, "attention: cache capacity %ld must be a multiple of 32", T_cap);
    if (q_stride < H * D || out_stride < H * D || q_stride % 8 || out_stride % 4)
        return set_error(SC_EINVAL, "attention: bad row strides");
    if (((uintptr_t)q | (uintptr_t)kc) % 16 || ((uintptr_t)vt | (uintptr_t)out) % 8)
        return set_error(SC_EINVAL, "attention: misaligned pointers");
    if (mask && (!ms || ms[0] < 0 || ms[1] < 0 || ms[2] < 0 || ms[3] < 0))
        return set_error(SC_EINVAL, "attention: mask strides must be given and non-negative");
    // many positions: attn_prefill_kernel (attn_prefill.hip, 128 columns a workgroup)
    // when the shape suits it; otherwise attn_kernel, which can also split the keys
    {
        const int pf = launch_attn_prefill(q, q_stride, kc, vt, T_cap, cache_len, out, out_stride, B, S, H, Hkv, D,
                                           scale, stream, mask, ms);
        if (pf <= 0) return pf;
    }
    AttnPlan pl;
    plan_attention(B, S, H, Hkv, D, T_cap, &pl);
    AttnArgs a = pl.a;
    a.q = q; a.q_stride = q_stride; a.kc = kc; a.vt = vt; a.cache_len = cache_len;
    a.out = out; a.out_stride = out_stride;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.part = nullptr;
    a.mask = mask;
    a.msb = mask ? ms[0] : 0; a.msh = mask ? ms[1] : 0; a.mss = mask ? ms[2] : 0; a.mst = mask ? ms[3] : 0;
    if (a.nsplit > 1) {
        const long need = B * H * S * (long)a.nsplit * (D + 4) * (long)sizeof(float);
        if (!workspace || workspace_bytes < need)
            return set_error(SC_EINVAL, "attention: workspace of %ld bytes required", need);
        if ((uintptr_t)workspace % 16) return set_error(SC_EINVAL, "attention: workspace must be 16-byte aligned");
        a.part = static_cast<float *>(workspace);
    }
    const unsigned blocks = (unsigned)pl.blocks;
    const dim3 grid(blocks), wg(64 * ATTN_WAVES);
    if (mask) {
        if (D == 128) hipLaunchKernelGGL((attn_kernel<128, true>), grid, wg, 0, stream, a);
        else hipLaunchKernelGGL((attn_kernel<64, true>), grid, wg, 0, stream, a);
    } else {
        if (D == 128) hipLaunchKernelGGL((attn_kernel<128, false>), grid, wg, 0, stream, a);
        else hipLaunchKernelGGL((attn_kernel<64, false>), grid, wg, 0, stream, a);
    }
    SC_HIP_CHECK(hipGetLastError());
    if (a.nsplit > 1) {
        const unsigned cb = (unsigned)((B * H * S + 3) / 4);
        if (D == 128) hipLaunchKernelGGL(attn_combine_kernel<128>, dim3(cb), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(attn_combine_kernel<64>, dim3(cb), dim3(256), 0, stream, a);
        SC_HIP_CHECK(hipGetLastError());
    }
    return SC_OK;
}

int launch_silu_mul(const uint16_t *gu, long rows, long I, uint16_t *out, hipStream_t stream) {
    if (!gu || !out) return set_error(SC_EINVAL, "silu_mul: null pointer");
    if (rows < 0 || I <= 0 || I % 8) return set_error(SC_EINVAL, "silu_mul: I=%ld must be a multiple of 8", I);
    if (((uintptr_t)gu | (uintptr_t)out) % 16) return set_error(SC_EINVAL, "silu_mul: pointers must be 16-byte aligned");
    if (rows == 0) return SC_OK;
    const long nv = rows * (I / 8);
    long blocks = (nv + 255) / 256;
    const long cap = 8L * device_info().num_cus;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, gu, out, rows, (int)I);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_argmax(const uint16_t *logits, long rows, long V, int32_t *ids, int32_t *tokens, long tok_stride,
                  long tok_cols, const int32_t *step, hipStream_t stream) {
    if (!logits || !ids) return set_error(SC_EINVAL, "argmax: null pointer");
    if (rows < 0 || V <= 0 || V > 0x7FFFFFFFL) return set_error(SC_EINVAL, "argmax: bad shape");
    if ((V % 8 == 0) && ((uintptr_t)logits % 16)) return set_error(SC_EINVAL, "argmax: logits must be 16-byte aligned");
    if (rows == 0) return SC_OK;
    if (tokens && (tok_cols < 1 || tok_stride < tok_cols)) return set_error(SC_EINVAL, "argmax: bad token buffer");
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, stream, logits, V, ids, tokens, tok_stride,
                       tok_cols, step);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_add_bf16(const uint16_t *a, const uint16_t *b, uint16_t *out, long n, hipStream_t stream) {
    if (!a || !b || !out) return set_error(SC_EINVAL, "add: null pointer");
    if (n < 0 || n % 8) return set_error(SC_EINVAL, "add: n=%ld must be a multiple of 8", n);
    if (((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) % 16) return set_error(SC_EINVAL, "add: pointers must be 16-byte aligned");
    if (n == 0) return SC_OK;
    long blocks = (n / 8 + 255) / 256;
    const long cap = 8L * device_info().num_cus;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(add_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a, b, out, n / 8);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

int launch_add_i32(int32_t *p, long n, int32_t delta, hipStream_t stream) {
    if (!p) return set_error(SC_EINVAL, "add_i32: null pointer");
    if (n < 0 || n > 64) return set_error(SC_EINVAL, "add_i32: n=%ld (at most 64 counters)", n);
    if (n == 0) return SC_OK;
    hipLaunchKernelGGL(add_i32_kernel, dim3(1), dim3(64), 0, stream, p, (int)n, delta);
    SC_HIP_CHECK(hipGetLastError());
    return SC_OK;
}

}  // namespace sc
