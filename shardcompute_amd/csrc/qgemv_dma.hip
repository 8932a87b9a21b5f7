// Kernel A (decode, M <= 8): persistent dequant-GEMV fed by LDS-DMA.
//
// y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// (mx.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits),
//  src/shardcompute/parallel/quantized_linear.py:168-176).
//
// Schedule (one workgroup per CU, 8 waves, or 4 when LDS is short):
// * Workgroup b owns the contiguous 16-column tiles [b*T/P, (b+1)*T/P) and
//   stages x (M rows, plus an all-zero row) and its per-group sums once.
// * Each wave walks a contiguous range of "items" = (tile, 256-byte chunk of
//   each of the tile's 16 weight rows) = 4 KB of packed weights (512 k for W4,
//   256 k for W8).  An item arrives by global_load_lds_dwordx4 straight into the
//   wave's LDS ring: 4 instructions of 4 rows x 256 contiguous bytes (fully
//   coalesced), plus one for the 16 rows' scales and biases.  No VGPRs hold data
//   in flight, so RING-1 items stay in flight while one is computed.
// * Each row is stored rotated by its row index (16-byte units), so the
//   MFMA-layout reads (16 rows, same column) hit 16 different bank groups.
// * The DMA is issued from inline asm and completion is awaited with explicit
//   vmcnt waits: the compiler cannot track LDS-DMA targets and would otherwise
//   wait for every outstanding load before any LDS read, serialising the ring.
// * Math is that of qgemv16.hip: codes become exact bf16 (W4: 128 + q through
//   the mantissa of 128.0; W8: q) as operand B of v_mfma_f32_16x16x32_bf16,
//   x is operand A, W4 spans use A-rows as selectors of the two quantization
//   groups, and acc += s * P + (b - off * s) * xsum[m, g].
// * Complete tiles are written from registers; a tile split between waves is
//   summed in wave order from per-wave LDS slots after a barrier, by the wave that
//   holds its last item (no atomics: results are reproducible run to run).
#include "dma_util.h"

namespace sc {

// What the kernel does to its input rows while staging them in LDS.
enum DmaPrologue {
    PRO_NONE = 0,   // x [M, K] as given
    PRO_NORM = 1,   // RMSNorm of x (+ res): the input layernorm before q|k|v, the
                    // post-attention layernorm before gate|up, the final norm before the lm_head
};

// What the kernel does with its output columns.
enum DmaEpilogue {
    EPI_NONE = 0,   // y [M, N]
    EPI_SWIGLU = 1, // the weight is gate|up stacked ([2I, K]); tile t pairs gate rows
                    // 8t..8t+7 with up rows I+8t..I+8t+7 and writes act = silu(g) * u
                    // [M, I] (parallel/mlp.py:241-245), never g and u themselves
};

struct DmaArgs {
    const uint16_t *x;
    const uint32_t *wq;
    const uint16_t *s;
    const uint16_t *b;
    const uint16_t *bias;
    uint16_t *y;
    int M, N, K, G;
    int max_tiles_per_block;
    int pro;
    const uint16_t *res;    // PRO_NORM: residual added first (may be null)
    const uint16_t *nw;     // PRO_NORM: norm weight [K]
    float eps;
    uint16_t *h_out;        // PRO_NORM with res: x + res, written by workgroup 0
    uint16_t *x_out;        // the staged input rows (normalised / gated), written by workgroup 0
    int dma_stage;          // input rows are staged by LDS-DMA (they fit the staging areas)
    int half;               // EPI_SWIGLU: I (rows of the gate half, output width)
};

namespace {

using namespace dma;
constexpr int DMA_MAX_WAVES = 8;
constexpr int XMAX = 8;                     // input chunks (16 B) per thread in the staging transform

}  // namespace

// MR: 1 for a single row of x (only D register 0 of lane-groups 0 and 2 matters),
// 8 for up to 8 rows.
template <int BITS, int MR, int PRO, int EPI>
__global__ void __launch_bounds__(64 * DMA_MAX_WAVES) qgemv_dma_kernel(DmaArgs a) {
    constexpr int NR = MR == 1 ? 1 : 4;                // D registers that can hold a row < M
    constexpr int SPAN_K = BITS == 4 ? 128 : 64;       // one 64-byte span of a row
    constexpr int SPAN_GROUPS = SPAN_K / 64;
    constexpr int SPAN_WORDS = SPAN_K / 8;
    constexpr int ITEM_K = 4 * SPAN_K;                 // 256 bytes of a row
    constexpr int ITEM_GROUPS = ITEM_K / 64;           // 8 (W4) / 4 (W8)
    constexpr int MFMAS = BITS == 4 ? 4 : 2;           // per span

    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int M = a.M, N = a.N, K = a.K, G = a.G;

    const int T = (N + 15) >> 4;
    const int P = gridDim.x;
    const int t_begin = (int)(blockIdx.x * (unsigned)T / (unsigned)P);       // T * P < 2^31 (host)
    const int t_end = (int)((blockIdx.x + 1) * (unsigned)T / (unsigned)P);
    const int ntl = t_end - t_begin;
    const int CPT = K / ITEM_K;
    const int items = ntl * CPT;
    const int W = K / 8;
    const int xstride = W + 1;

    // LDS carve-up: rings | x (M rows + zero row) | xsum | split-tile partials | bias
    uint8_t *ring = smem + (size_t)wave * RING * SLOT_BYTES;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring;
    uint4 *xl = reinterpret_cast<uint4 *>(smem + (size_t)nwaves * RING * SLOT_BYTES);
    float *xs = reinterpret_cast<float *>(xl + (size_t)(M + 1) * xstride);
    // a wave's range splits at most two tiles (its first and its last): one partial
    // slot each; the last contributor to arrive sums the slots in wave order, so
    // results are reproducible without a barrier
    float *part_l = xs + M * G;
    // the bias slice lives in LDS: a global load inside the ring loop would make the
    // compiler wait for every outstanding DMA
    uint16_t *bias_l = reinterpret_cast<uint16_t *>(part_l + (size_t)nwaves * 2 * M * 16);
    int *cnt = reinterpret_cast<int *>(bias_l + ((a.max_tiles_per_block * 16 + 1) & ~1));   // items summed per tile

    // waves split the items evenly; 4 or 8 waves, so the division is a shift (a
    // 64-bit or variable division costs a software routine on every use)
    const int nwl2 = 31 - __clz(nwaves);
    const int lo = (wave * items) >> nwl2;
    const int hi = ((wave + 1) * items) >> nwl2;

    // ---- item DMA: 4 x (4 rows x 256 B, row-rotated) + scales/biases of the 16 rows.
    // Pointers advance incrementally; they are rebuilt only when the tile changes.
    const size_t row_bytes = (size_t)K * BITS / 8;
    int iss_tl = lo / CPT, iss_ch = lo - (lo / CPT) * CPT, iss_left = hi - lo;
    const uint8_t *gw[4];
    const uint16_t *gsb = nullptr;
    // weight row of row r (0..15) of the tile that starts at output column n0
    auto wrow = [&](int n0, int r) -> int {
        if (EPI == EPI_SWIGLU) return (r < 8 ? 0 : a.half - 8) + (n0 >> 1) + r;
        return min(n0 + r, N - 1);
    };
    auto set_tile = [&](int tl) {
        const int n0 = (t_begin + tl) * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * i + (lane >> 4);
            const int col = ((lane & 15) - r) & 15;
            gw[i] = reinterpret_cast<const uint8_t *>(a.wq) + (size_t)wrow(n0, r) * row_bytes + col * 16;
        }
        gsb = (lane < 16 ? a.s : a.b) + (size_t)wrow(n0, j) * G;
    };
    set_tile(iss_tl);
    auto issue = [&](int slot) {
        const uint32_t dst = ring_lds + slot * SLOT_BYTES;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(gw[i] + (size_t)iss_ch * 256, dst + i * 1024);
        // scales: lanes 0-15 -> row j; biases: lanes 16-31 -> row j (8 groups, 16 B)
        if (lane < 32) dma16(gsb + ((iss_ch * ITEM_GROUPS) & ~7), dst + SLOT_W);
        // advance to the next item; past the end the last item is loaded again
        if (iss_left > 1) {
            --iss_left;
            if (++iss_ch == CPT) {
                iss_ch = 0;
                set_tile(++iss_tl);
            }
        }
    };

    // ---- input rows.  Every workgroup stages the same rows with the same arithmetic,
    // so a fused normalisation or gate yields identical inputs in all of them (and
    // the same bits as the standalone kernels, which share the math and the row
    // partition: 256 threads per row, thread t holding chunks t, t + 256, ...).
    // When they fit, the raw rows arrive by LDS-DMA issued before the weight ring
    // starts: x (or gate|up) into the x area, residual and norm weight into the
    // third ring slot of every wave (idle until the ring loop), and only they are
    // waited for.  Otherwise (and for linears with a bias) ordinary loads stage
    // them, which the compiler waits for together with the weight DMA.
    const bool has_work = hi > lo;
    const bool dstage = PRO == PRO_NONE && a.dma_stage != 0;   // (the norm prologue stages with ordinary loads)
    const int groups = blockDim.x / NORM_THREADS;
    const int gsel = tid / NORM_THREADS, tg = tid - gsel * NORM_THREADS;
    const int WPT = (W + NORM_THREADS - 1) / NORM_THREADS;    // norm chunks per row and thread
    const uint32_t xraw = (uint32_t)(uintptr_t)xl;
    auto s2_unit = [&](int u) -> uint32_t {
        return (uint32_t)(uintptr_t)(smem + (size_t)(u / S2_UNITS) * RING * SLOT_BYTES + 2 * SLOT_BYTES +
                                     (size_t)(u % S2_UNITS) * 1024);
    };
    const int ru = (int)(((size_t)M * K * 2 + 1023) / 1024);   // staging units of the residual rows
    if (dstage) {
        auto stage = [&](const uint16_t *src, size_t bytes, int unit0, bool to_s2) {
            const int units = (int)((bytes + 1023) / 1024);
            for (int u = wave; u < units; u += nwaves) {
                const size_t off = (size_t)u * 1024 + 16 * lane;
                const uint32_t dst = to_s2 ? s2_unit(unit0 + u) : xraw + (uint32_t)u * 1024;
                if (off < bytes) dma16(reinterpret_cast<const uint8_t *>(src) + off, dst);
            }
        };
        stage(a.x, (size_t)M * K * 2, 0, false);
        if (PRO == PRO_NORM) {
            if (a.res) stage(a.res, (size_t)M * K * 2, 0, true);
            stage(a.nw, (size_t)K * 2, ru, true);
        }
    }
    if (has_work) {
#pragma unroll
        for (int k = 0; k < RING - 1; ++k) issue(k);
    }
    if (dstage) {
        if (has_work) wait_vm<DMA_PER_ITEM * (RING - 1)>();
        else wait_vm<0>();
        __syncthreads();
        const uint4 *raw = reinterpret_cast<const uint4 *>(xl);
        auto s2_chunk = [&](size_t chunk) -> uint4 {      // 16-byte chunk of the ring-slot staging area
            const size_t bo = chunk * 16;
            return *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(smem) +
                                                    (s2_unit((int)(bo / 1024)) - (uint32_t)(uintptr_t)smem) +
                                                    bo % 1024);
        };
        uint4 v[XMAX];
        if (PRO == PRO_NORM) {
            __shared__ float red[8][NORM_THREADS / 64];
            __shared__ float root_l[8];
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < XMAX; ++i) {
                const int ri = i / WPT, m = gsel + groups * ri, w = tg + NORM_THREADS * (i - ri * WPT);
                const bool ok = m < M && w < W && ri * groups < M;
                if (ok) {
                    v[i] = raw[m * W + w];
                    if (a.res) {
                        v[i] = add_bf16x8(v[i], s2_chunk((size_t)m * W + w));
                        if (blockIdx.x == 0 && a.h_out)
                            *reinterpret_cast<uint4 *>(a.h_out + (size_t)m * K + (size_t)w * 8) = v[i];
                    }
                    ss = sumsq_bf16x8(ss, v[i]);
                }
                if ((i % WPT) == WPT - 1 || i == XMAX - 1) {      // end of this thread's chunks of a row
                    const float tot = wave_sum(ss);
                    if (m < M && (tg & 63) == 0) red[m][tg >> 6] = tot;
                    ss = 0.f;
                }
            }
            __syncthreads();                                        // raw x fully read: the area is reused below
            if (tid < M) {
                float tot = 0.f;
#pragma unroll
                for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[tid][i];
                root_l[tid] = rms_root(tot, K, a.eps);
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < XMAX; ++i) {
                const int ri = i / WPT, m = gsel + groups * ri, w = tg + NORM_THREADS * (i - ri * WPT);
                if (m < M && w < W && ri * groups < M) {
                    const uint4 o = norm_bf16x8(v[i], s2_chunk((size_t)ru * 64 + w), root_l[m]);
                    if (blockIdx.x == 0 && a.x_out) *reinterpret_cast<uint4 *>(a.x_out + (size_t)m * K + (size_t)w * 8) = o;
                    xl[m * xstride + w] = BITS == 4 ? perm_w4x(o) : o;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < XMAX; ++i) {
                const int idx = tid + i * (int)blockDim.x;
                if (idx < M * W) v[i] = raw[idx];
            }
            __syncthreads();                                        // raw rows fully read
#pragma unroll
            for (int i = 0; i < XMAX; ++i) {
                const int idx = tid + i * (int)blockDim.x;
                if (idx < M * W) {
                    const int m = idx / W, w = idx - (idx / W) * W;
                    xl[m * xstride + w] = BITS == 4 ? perm_w4x(v[i]) : v[i];
                }
            }
        }
    } else if (PRO == PRO_NONE) {
        for (int idx = tid; idx < M * W; idx += blockDim.x) {
            const int m = idx / W, w = idx - (idx / W) * W;
            const uint4 v = *reinterpret_cast<const uint4 *>(a.x + (size_t)m * K + (size_t)w * 8);
            xl[m * xstride + w] = BITS == 4 ? perm_w4x(v) : v;
        }
    } else {
        __shared__ float red[8][NORM_THREADS / 64];
        __shared__ float root_l[8];
        for (int idx = tid; idx < M * W; idx += blockDim.x) {
            const int m = idx / W, w = idx - (idx / W) * W;
            uint4 v = *reinterpret_cast<const uint4 *>(a.x + (size_t)m * K + (size_t)w * 8);
            if (a.res) {
                v = add_bf16x8(v, *reinterpret_cast<const uint4 *>(a.res + (size_t)m * K + (size_t)w * 8));
                if (blockIdx.x == 0 && a.h_out) *reinterpret_cast<uint4 *>(a.h_out + (size_t)m * K + (size_t)w * 8) = v;
            }
            xl[m * xstride + w] = v;
        }
        __syncthreads();
        // per-row sums of squares, 256 threads per row as in the standalone RMSNorm
        const int groups = blockDim.x / NORM_THREADS;
        const int gsel = tid / NORM_THREADS, t = tid - gsel * NORM_THREADS;
        for (int m0 = 0; m0 < M; m0 += groups) {
            const int m = m0 + gsel;
            if (m < M) {
                float ss = 0.f;
                for (int idx = t; idx < W; idx += NORM_THREADS) ss = sumsq_bf16x8(ss, xl[m * xstride + idx]);
                ss = wave_sum(ss);
                if ((t & 63) == 0) red[m][t >> 6] = ss;
            }
        }
        __syncthreads();
        if (tid < M) {
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[tid][i];
            root_l[tid] = rms_root(tot, K, a.eps);
        }
        __syncthreads();
        for (int idx = tid; idx < M * W; idx += blockDim.x) {
            const int m = idx / W, w = idx - (idx / W) * W;
            const uint4 v = norm_bf16x8(xl[m * xstride + w], reinterpret_cast<const uint4 *>(a.nw)[w], root_l[m]);
            if (blockIdx.x == 0 && a.x_out) *reinterpret_cast<uint4 *>(a.x_out + (size_t)m * K + (size_t)w * 8) = v;
            xl[m * xstride + w] = BITS == 4 ? perm_w4x(v) : v;
        }
    }
    if (a.bias)
        for (int idx = tid; idx < ntl * 16; idx += blockDim.x)
            bias_l[idx] = a.bias[wrow((t_begin + (idx >> 4)) * 16, idx & 15)];
    for (int idx = tid; idx < W; idx += blockDim.x) xl[M * xstride + idx] = make_uint4(0u, 0u, 0u, 0u);
    for (int idx = tid; idx < ntl; idx += blockDim.x) cnt[idx] = 0;
    __syncthreads();
    for (int idx = tid; idx < M * G; idx += blockDim.x) {
        const int m = idx / G, g = idx - (idx / G) * G;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint4 v = xl[m * xstride + g * 8 + w];
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += bf2f(wh(v, e));
        }
        xs[m * G + g] = sum;
    }
    __syncthreads();

    // A operand rows (zero row for lanes that carry no x) and D-row mapping
    const int am = (BITS == 4) ? (j & 7) : j;
    const bool a_on = (am < M) && (BITS == 8 || (j >> 3) == (q >> 1));
    const uint4 *xrow = xl + min(am, M - 1) * xstride;
    const int epar = (BITS == 4) ? (q >> 1) : 0;
    const int em0 = (BITS == 4) ? 4 * (q & 1) : 4 * q;

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    int cur_tile = lo / CPT, chunks_in_acc = 0;
    // bf16 128.0 in both halves, kept in a VGPR for v_and_or_b32
    uint32_t magic = 0x43004300u;
    asm volatile("" : "+v"(magic));
    uint32_t nib_mask = 0x000F000Fu;
    asm volatile("" : "+s"(nib_mask));

    auto write_out = [&](int tl, int m, int jj, float v) {
        const int nn = (t_begin + tl) * 16 + jj;
        if (nn < N && m < M) {
            uint32_t o = f2bf(v);
            if (a.bias) o = f2bf(bf2f(o) + bf2f(bias_l[tl * 16 + jj]));
            a.y[(size_t)m * N + nn] = (uint16_t)o;
        }
    };
    // gate (jg) and up (jg + 8) columns of a paired tile -> act column 8 * tile + jg
    auto write_act = [&](int tl, int m, int jg, float vg, float vu) {
        if (m < M) {
            uint32_t gb = f2bf(vg), ub = f2bf(vu);
            if (a.bias) {
                gb = f2bf(bf2f(gb) + bf2f(bias_l[tl * 16 + jg]));
                ub = f2bf(bf2f(ub) + bf2f(bias_l[tl * 16 + 8 + jg]));
            }
            a.y[(size_t)m * a.half + (size_t)(t_begin + tl) * 8 + jg] = (uint16_t)f2bf(silu_mul_f(bf2f(gb), bf2f(ub)));
        }
    };
    int fin_a = -1, fin_b = -1;      // split tiles this wave completes
    auto flush = [&]() {
        f4 fin = acc;
        if (BITS == 4) {
#pragma unroll
            for (int r = 0; r < 4; ++r) fin[r] += __shfl_xor(fin[r], 32);
        }
        if (chunks_in_acc == CPT) {
            if (EPI == EPI_SWIGLU) {
                f4 up;
#pragma unroll
                for (int r = 0; r < 4; ++r) up[r] = __shfl_xor(fin[r], 8);   // column j + 8 of the same rows
                if (q < 2 && j < 8) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) write_act(cur_tile, em0 + r, j, fin[r], up[r]);
                }
            } else if (q < 2) {
#pragma unroll
                for (int r = 0; r < 4; ++r) write_out(cur_tile, em0 + r, j, fin[r]);
            }
        } else {
            if (q < 2) {
                float *pl = part_l + ((size_t)wave * 2 + (cur_tile == lo / CPT ? 0 : 1)) * M * 16;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (em0 + r < M) pl[(em0 + r) * 16 + j] = fin[r];
            }
            wait_lgkm0();                                       // slot written before the count
            int done = 0;
            if (lane == 0) done = (atomicAdd(&cnt[cur_tile], chunks_in_acc) + chunks_in_acc) == CPT;
            done = __shfl(done, 0);
            // the last contributor sums the tile after its ring loop (keeps the loop short)
            if (done) {
                if (fin_a < 0) fin_a = cur_tile;
                else fin_b = cur_tile;
            }
        }
        acc = f4{0.f, 0.f, 0.f, 0.f};
        chunks_in_acc = 0;
    };

    auto compute = [&](int itc, int slot) {
        const int tl = itc / CPT, ch = itc - (itc / CPT) * CPT;
        if (tl != cur_tile) {
            flush();
            cur_tile = tl;
        }
        const uint4 *sl = reinterpret_cast<const uint4 *>(ring + slot * SLOT_BYTES);
        // weights of row j, span t, 16-byte column (4t + q), stored rotated by j
        uint4 wv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) wv[t] = sl[(j >> 2) * 64 + (j & 3) * 16 + ((4 * t + q + j) & 15)];
        const uint4 sv = sl[SLOT_W / 16 + j];
        const uint4 bv = sl[SLOT_W / 16 + 16 + j];
        const int gsub = (ch * ITEM_GROUPS) & 7;   // first group of this item inside the 8 loaded
        // x operand: only lanes whose A-row carries x read LDS (exec-masked); the
        // rest multiply zeros
        uint4 xa[4][MFMAS];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int u = 0; u < MFMAS; ++u) xa[t][u] = make_uint4(0u, 0u, 0u, 0u);
        if (a_on) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int u = 0; u < MFMAS; ++u)
                    xa[t][u] = xrow[(ch * 4 + t) * SPAN_WORDS + (BITS == 4 ? 4 * q + u : 2 * q + u)];
        }
        float xsv[4][NR];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int g = (ch * 4 + t) * SPAN_GROUPS + epar;
#pragma unroll
            for (int r = 0; r < NR; ++r) xsv[t][r] = xs[min(em0 + r, M - 1) * G + g];
        }
        // four independent MFMA chains (one per span), interleaved to hide MFMA latency
        f4 P[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) P[t] = f4{0.f, 0.f, 0.f, 0.f};
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
                P[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[t][u]), B, P[t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int gsel = gsub + t * SPAN_GROUPS + epar;
            const float sf = bf2f(wh(sv, gsel));
            const float bf = bf2f(wh(bv, gsel));
            const float cf = BITS == 4 ? fmaf(-128.f, sf, bf) : bf;
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r] = fmaf(sf, P[t][r], fmaf(cf, xsv[t][r], acc[r]));
        }
        ++chunks_in_acc;
    };

    // ---- ring: item lo+i sits in slot i % RING; RING-1 items are always in flight
    if (has_work) {
        const int n_my = hi - lo;
        int i = 0;
        for (; i + RING <= n_my; i += RING) {
#pragma unroll
            for (int k = 0; k < RING; ++k) {
                issue((k + RING - 1) % RING);
                wait_vm<DMA_PER_ITEM * (RING - 1)>();
                compute(lo + i + k, k);
            }
        }
        for (int k = 0; i < n_my; ++i, ++k) {
            issue((k + RING - 1) % RING);
            wait_vm<DMA_PER_ITEM * (RING - 1)>();
            compute(lo + i, k % RING);
        }
        flush();
    }
    wait_vm<0>();
    // ---- split tiles whose last contributor this wave was: sum the partial slots in
    // wave order (every contributor wrote its slot before counting itself)
    for (int f = 0; f < 2; ++f) {
        const int tile = f == 0 ? fin_a : fin_b;
        if (tile < 0) continue;
        wait_lgkm0();
        const int ts = tile * CPT, te = ts + CPT;
        auto slot_sum = [&](int o) {
            float v = 0.f;
            for (int w2 = 0; w2 < nwaves; ++w2) {
                const int lo2 = (w2 * items) >> nwl2, hi2 = ((w2 + 1) * items) >> nwl2;
                if (hi2 <= lo2 || hi2 <= ts || lo2 >= te) continue;
                v += part_l[((size_t)w2 * 2 + (lo2 / CPT == tile ? 0 : 1)) * M * 16 + o];
            }
            return v;
        };
        if (EPI == EPI_SWIGLU) {
            for (int o = lane; o < M * 8; o += 64)
                write_act(tile, o >> 3, o & 7, slot_sum((o >> 3) * 16 + (o & 7)), slot_sum((o >> 3) * 16 + 8 + (o & 7)));
        } else {
            for (int o = lane; o < M * 16; o += 64) write_out(tile, o >> 4, o & 15, slot_sum(o));
        }
    }
}

// ---------------------------------------------------------------- host side

int launch_qgemv_m1(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                    const uint16_t *bias, uint16_t *y, int N, int K, int bits, hipStream_t stream,
                    const DmaFused *fused);

bool qgemv_dma_eligible(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b, int M, int K) {
    (void)x;
    return M >= 1 && M <= 8 && K % 512 == 0 && !((uintptr_t)s % 16) && !((uintptr_t)b % 16) && !((uintptr_t)wq % 16);
}

int launch_qgemv_dma(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                     const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits, hipStream_t stream,
                     const DmaFused *fused) {
    if (M < 1 || M > 8) return SC_EUNSUPPORTED;
    const bool head = fused && fused->head;             // greedy selection: the batch-1 kernel only
    if (head && M != 1) return SC_EUNSUPPORTED;
    if (M == 1) {       // batch 1: the dynamically balanced kernel (qgemv_m1.hip) when it applies
        const int rc = launch_qgemv_m1(x, wq, s, b, bias, y, N, K, bits, stream, fused);
        if (rc != SC_EUNSUPPORTED || head) return rc;
    }
    if (K % 512) return SC_EUNSUPPORTED;                       // 16-byte aligned scale rows, whole items
    if (((uintptr_t)s % 16) || ((uintptr_t)b % 16) || ((uintptr_t)wq % 16)) return SC_EUNSUPPORTED;
    const DeviceInfo &di = device_info();
    const int item_k = bits == 4 ? 512 : 256;
    const int T = (N + 15) / 16;
    const int CPT = K / item_k;
    const int G = K / 64;
    const int lds_cap = di.max_lds_per_block < 160 * 1024 ? di.max_lds_per_block : 160 * 1024;
    // 8 waves per CU when their rings fit LDS next to x, else 4
    int waves = 0, P = 0;
    size_t lds = 0;
    for (int w = DMA_MAX_WAVES; w >= 4; w /= 2) {
        P = di.num_cus;
        while (P > 1 && (long)T * CPT < (long)P * w) P /= 2;
        const int tpb = (T + P - 1) / P;
        lds = (size_t)w * RING * SLOT_BYTES + (size_t)(M + 1) * (K / 8 + 1) * 16 + (size_t)M * G * 4 +
              (size_t)w * 2 * M * 16 * 4 + (size_t)tpb * 16 * 2 + 4 + (size_t)tpb * 4;
        if (lds + 256 <= (size_t)lds_cap) { waves = w; break; }   // + the norm prologue's static LDS
    }
    if (!waves) return SC_EUNSUPPORTED;
    const int max_tpb = (T + P - 1) / P;
    // the kernel's tile and item ranges use 32-bit products
    if ((long)T * P >= (1L << 31) || (long)max_tpb * CPT * DMA_MAX_WAVES >= (1L << 31)) return SC_EUNSUPPORTED;
    DmaArgs a;
    a.x = x; a.wq = wq; a.s = s; a.b = b; a.bias = bias; a.y = y;
    a.M = M; a.N = N; a.K = K; a.G = G; a.max_tiles_per_block = max_tpb;
    a.pro = PRO_NONE; a.res = nullptr; a.nw = nullptr; a.eps = 0.f; a.h_out = nullptr; a.x_out = nullptr;
    a.half = 0;
    int epi = EPI_NONE;
    if (fused) {
        a.pro = fused->kind; a.res = fused->res; a.nw = fused->norm_weight; a.eps = fused->eps;
        a.h_out = fused->h_out; a.x_out = fused->x_out;
        if (fused->swiglu_half > 0) {
            if (fused->swiglu_half % 8 || N != 2 * fused->swiglu_half) return SC_EUNSUPPORTED;
            epi = EPI_SWIGLU;
            a.half = fused->swiglu_half;
        }
    }
    {
        // LDS-DMA staging needs 16-byte rows, the raw rows within the x area, the
        // residual and norm weight within the waves' third ring slots, and at most
        // XMAX chunks per thread in the transform
        const int threads = 64 * waves, W = K / 8;
        const int groups = threads / NORM_THREADS;
        const size_t x_area = (size_t)(M + 1) * (W + 1) * 16;
        const size_t s2_area = (size_t)waves * S2_UNITS * 1024;
        // (measured: the norm prologue is faster with ordinary loads)
        bool ok = !bias && !((uintptr_t)x % 16) && a.pro == PRO_NONE;
        const int chunks = (M * W + threads - 1) / threads;
        ok = ok && chunks <= XMAX && (size_t)M * K * 2 <= x_area;
        (void)groups;
        (void)s2_area;
        a.dma_stage = ok;
    }
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
    // one instantiation per prologue and epilogue keeps each kernel's code short
    // (these launches are latency-bound, and a cold instruction fetch of unused code
    // shows)
    static int cfg[2][2][2][2] = {};
    const int bi = bits == 4 ? 0 : 1, mi = M == 1 ? 0 : 1, pi = a.pro;
    int &c = cfg[bi][mi][pi][epi];
#define SC_DMA_PICK(B_, M_)                                                                        \
    do {                                                                                            \
        if (pi == PRO_NORM && epi == EPI_SWIGLU) return launch(qgemv_dma_kernel<B_, M_, PRO_NORM, EPI_SWIGLU>, c); \
        if (pi == PRO_NORM) return launch(qgemv_dma_kernel<B_, M_, PRO_NORM, EPI_NONE>, c);        \
        if (epi == EPI_SWIGLU) return launch(qgemv_dma_kernel<B_, M_, PRO_NONE, EPI_SWIGLU>, c);   \
        return launch(qgemv_dma_kernel<B_, M_, PRO_NONE, EPI_NONE>, c);                            \
    } while (0)
    if (bits == 4) {
        if (M == 1) SC_DMA_PICK(4, 1);
        SC_DMA_PICK(4, 8);
    }
    if (M == 1) SC_DMA_PICK(8, 1);
    SC_DMA_PICK(8, 8);
#undef SC_DMA_PICK
}

}  // namespace sc
