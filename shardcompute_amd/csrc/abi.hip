// C-ABI of libshardcompute_hip: argument checks, dispatch, error reporting and
// the library-owned split-K scratch.  Declarations live in
// include/shardcompute_hip.h, which cites the reference call each entry replaces.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "sc_common.h"
#include "../../include/shardcompute_hip.h"

namespace sc {

int launch_qgemv_dma(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                     const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits, hipStream_t stream,
                     const DmaFused *fused = nullptr);
bool qgemv_dma_eligible(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b, int M, int K);
int launch_qgemv16(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b, const uint16_t *bias,
                   uint16_t *y, int M, int N, int K, int bits, hipStream_t stream, bool no_alloc, int swiglu_half = 0,
                   SplitKeep *keep = nullptr);
int launch_qgemv_skinny(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                        const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits, hipStream_t stream);
int launch_qgemm_mfma(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                      const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits, hipStream_t stream,
                      int swiglu_half = 0, bool no_alloc = false);
int launch_qgemm_band(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                      const uint16_t *bias, uint16_t *y, int M, int N, int K, int bits, hipStream_t stream,
                      bool no_alloc, int swiglu_half, int force_nw, int force_split, SplitKeep *keep = nullptr);
int launch_vocab_gather(const void *ids, int ids_is_int64, int64_t T, const uint16_t *table, int64_t v_local,
                        int64_t D, int64_t vocab_start, uint16_t *out, hipStream_t stream);
int launch_qembed_gather(const void *ids, int ids_is_int64, int64_t T, const uint32_t *wq, const uint16_t *s,
                         const uint16_t *b, int64_t v_local, int64_t D, int64_t vocab_start, int bits,
                         uint16_t *out, hipStream_t stream);
int launch_quantize(const float *w, int64_t rows, int64_t K, int bits, uint32_t *wq, uint16_t *s, uint16_t *b,
                    hipStream_t stream);
int launch_dequantize(const uint32_t *wq, const uint16_t *s, const uint16_t *b, int64_t rows, int64_t K, int bits,
                      uint16_t *out, hipStream_t stream);

int launch_split_add_rms_norm(const float *partials, int splits, const uint16_t *y_in, const uint16_t *bias,
                              const uint16_t *res, const uint16_t *w, uint16_t *h_out, uint16_t *out, long rows, long D,
                              float eps, hipStream_t stream);
int launch_rms_norm(const uint16_t *x, const uint16_t *res, const uint16_t *w, uint16_t *y, uint16_t *h_out,
                    long rows, long D, float eps, hipStream_t stream);
int launch_rope_append(uint16_t *qkv, long qkv_stride, long B, long S, long H, long Hkv, long D,
                       const float *cos_t, const float *sin_t, long table_len, uint16_t *kc, uint16_t *vt,
                       long T_cap, const int32_t *cache_len, long pos_offset, hipStream_t stream);
long attention_workspace_bytes(long B, long S, long H, long Hkv, long D, long T_cap);
long attention_decode_workspace_bytes(long B, long H, long Hkv, long D, long T_cap);
int launch_attention_decode(const uint16_t *qkv, long qkv_stride, long B, long H, long Hkv, long D,
                            const float *cos_t, const float *sin_t, long table_len, uint16_t *kc, uint16_t *vt,
                            long T_cap, const int32_t *cache_len, long pos_offset, float scale, uint16_t *out,
                            long out_stride, void *workspace, long workspace_bytes, hipStream_t stream,
                            const float *mask = nullptr, const long *ms = nullptr);
int launch_attention(const uint16_t *q, long q_stride, const uint16_t *kc, const uint16_t *vt, long T_cap,
                     const int32_t *cache_len, uint16_t *out, long out_stride, long B, long S, long H, long Hkv,
                     long D, float scale, void *workspace, long workspace_bytes, hipStream_t stream,
                     const float *mask, const long *mask_strides);
int launch_silu_mul(const uint16_t *gu, long rows, long I, uint16_t *out, hipStream_t stream);
int launch_argmax(const uint16_t *logits, long rows, long V, int32_t *ids, int32_t *tokens, long tok_stride,
                  long tok_cols, const int32_t *step, hipStream_t stream);
int launch_add_bf16(const uint16_t *a, const uint16_t *b, uint16_t *out, long n, hipStream_t stream);
int launch_add_i32(int32_t *p, long n, int32_t delta, hipStream_t stream);
int decode_plan_create(const sc_decode_model *m, const sc_decode_layer *layers, void **out);
int decode_plan_run(void *plan, hipStream_t stream);
int decode_plan_status(void *plan, unsigned *status);
int decode_plan_trace(void *plan, int enable);
int decode_plan_read_trace(void *plan, uint32_t *host, int64_t n, int *P, int *nops);
void decode_plan_destroy(void *plan);

constexpr int PRO_NORM_KIND = 1;

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

static constexpr int kMaxDevices = 64;
static std::mutex g_mu;
static DeviceInfo g_info[kMaxDevices];
static bool g_info_ok[kMaxDevices];

struct ScratchSlot {
    float *partials = nullptr;
    unsigned *counters = nullptr;
    size_t partial_cap = 0;
    size_t counter_cap = 0;
};
static ScratchSlot g_scratch[kMaxDevices];

const DeviceInfo &device_info() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
    if (!g_info_ok[dev]) {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_info_ok[dev]) {
            DeviceInfo di;
            int v = 0;
            di.num_cus = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? v : 256;
            di.max_lds_per_block =
                hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess ? v : 65536;
            g_info[dev] = di;
            g_info_ok[dev] = true;
        }
    }
    return g_info[dev];
}

// Grows (never shrinks) the calling device's split-K scratch.  Counters must
// start at zero; the kernels return every counter they use to zero.  Growing
// synchronises the device so no in-flight kernel still uses the old buffers.
int splitk_scratch(size_t partial_floats, size_t n_counters, SplitKScratch *out) {
    int dev = 0;
    SC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return set_error(SC_EINVAL, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_mu);
    ScratchSlot &sl = g_scratch[dev];
    if (sl.partial_cap < partial_floats || sl.counter_cap < n_counters) {
        const size_t pc = partial_floats > sl.partial_cap ? partial_floats : sl.partial_cap;
        const size_t cc = n_counters > sl.counter_cap ? n_counters : sl.counter_cap;
        SC_HIP_CHECK(hipDeviceSynchronize());
        if (sl.partials) SC_HIP_CHECK(hipFree(sl.partials));
        if (sl.counters) SC_HIP_CHECK(hipFree(sl.counters));
        sl.partials = nullptr;
        sl.counters = nullptr;
        sl.partial_cap = sl.counter_cap = 0;
        SC_HIP_CHECK(hipMalloc(&sl.partials, pc * sizeof(float)));
        SC_HIP_CHECK(hipMalloc(&sl.counters, cc * sizeof(unsigned)));
        SC_HIP_CHECK(hipMemset(sl.counters, 0, cc * sizeof(unsigned)));
        SC_HIP_CHECK(hipDeviceSynchronize());
        sl.partial_cap = pc;
        sl.counter_cap = cc;
    }
    out->partials = sl.partials;
    out->counters = sl.counters;
    return SC_OK;
}

static bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

static int check_qmm(const void *x, const void *wq, const void *s, const void *b, const void *y, int64_t M,
                     int64_t N, int64_t K, int bits, int group_size) {
    if (!x || !wq || !s || !b || !y) return set_error(SC_EINVAL, "qmm: null pointer argument");
    if (bits != 4 && bits != 8) return set_error(SC_EUNSUPPORTED, "qmm: bits=%d (supported: 4, 8)", bits);
    if (group_size != 64) return set_error(SC_EUNSUPPORTED, "qmm: group_size=%d (supported: 64)", group_size);
    if (M < 1 || N < 1 || K < 1) return set_error(SC_EINVAL, "qmm: empty shape M=%lld N=%lld K=%lld",
                                                  (long long)M, (long long)N, (long long)K);
    if (K % group_size) return set_error(SC_EINVAL, "qmm: K=%lld not a multiple of group_size=%d", (long long)K,
                                         group_size);
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
        return set_error(SC_EINVAL, "qmm: dimension above 2^30");
    if (!aligned(x, 16) || !aligned(wq, 16))
        return set_error(SC_EINVAL, "qmm: x and wq must be 16-byte aligned");
    if (!aligned(s, 2) || !aligned(b, 2) || !aligned(y, 2))
        return set_error(SC_EINVAL, "qmm: scales, biases and y must be 2-byte aligned");
    return SC_OK;
}

// Whether the automatic choice is the band kernel: 33-160 rows (measured faster than
// the GEMM's 256-row tiles up to 128 rows, slower at 256); 17-32 rows, where both
// kernels compute 32 rows and the band's stream is the faster (8B gate|up at 20, 24
// and 32 rows 28, 31, 30 against 32, 34, 34 us on the GEMV; the 8B lm_head at 32 rows
// 99 against 119 us); 9-16 rows where the 16-column GEMV's K splits or x staging cost
// more than the band's stream: K above 4096 or at most 8192 weight rows (8B down at 16
// rows 17 against 25 us; 8B gate|up at 16 rows 29 against 24 us and the lm_head 95
// against 73 us stay on the GEMV, which computes 16 rows where the band computes 32);
// and 8 rows with K of 4096 or more (8B q|k|v, gate|up, down 10, 15, 16 against 12,
// 17, 26 us on the 8-row GEMV; K = 2048 is a tie).
static bool band_first(int64_t M, int64_t N, int64_t K) {
    if (M > 32) return M <= 160;
    if (M == 8) return K >= 4096;
    return M > 16 || (M > 8 && (K > 4096 || N <= 8192));
}

static int qmm_dispatch(const uint16_t *x, const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                        const uint16_t *bias, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                        int group_size, void *stream, int path, bool no_alloc = false, SplitKeep *keep = nullptr) {
    int rc = check_qmm(x, wq, s, b, y, M, N, K, bits, group_size);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (path == SC_QMM_PATH_AUTO) path = band_first(M, N, K) ? SC_QMM_PATH_BAND : M <= 32 ? SC_QMM_PATH_GEMV
                                                                                    : SC_QMM_PATH_GEMM;
    if (path == SC_QMM_PATH_BAND) {
        // any M <= 256: the weight-streaming band kernel; shapes it does not take (K not
        // a multiple of 512, partials beyond the no-alloc scratch) go to the GEMVs up to
        // 32 rows, to the GEMM above
        rc = launch_qgemm_band(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, no_alloc, 0, 0, 0, keep);
        if (rc != SC_EUNSUPPORTED) return rc;
        if (M > 32) return launch_qgemm_mfma(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, 0, no_alloc);
        path = SC_QMM_PATH_GEMV;
    }
    if (path == SC_QMM_PATH_GEMV) {
        // M <= 8: persistent LDS-DMA GEMV; otherwise (or when x does not fit its
        // LDS) the 16-column split-K GEMV; K not a multiple of 512 (W4) / 256 (W8)
        // takes the 32-column generic-K kernel; x that fits no LDS layout, the GEMM
        rc = launch_qgemv_dma(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st);
        if (rc != SC_EUNSUPPORTED) return rc;
        rc = launch_qgemv16(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, no_alloc, 0, keep);
        if (rc != SC_EUNSUPPORTED) return rc;
        rc = launch_qgemv_skinny(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st);
        if (rc != SC_EUNSUPPORTED) return rc;
        return launch_qgemm_mfma(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, 0, no_alloc);
    }
    if (path == SC_QMM_PATH_GEMM)
        return launch_qgemm_mfma(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, 0, no_alloc);
    return set_error(SC_EINVAL, "qmm: unknown path %d", path);
}

static bool overlap(const void *a, size_t an, const void *b, size_t bn) {
    if (!a || !b) return false;
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + bn && y < x + an;
}

// The quantized product of a transformed input and/or with a transformed output:
//  * nw != null: the input is RMSNorm(x + res) (res optional), left in x_out and,
//    with res, x + res in h_out;
//  * swiglu_half > 0: the weight is gate|up stacked [2I, K] and y receives
//    act = silu(gate) * up [M, I] (gu_scratch [M, 2I] holds the product when the
//    fused kernel does not apply).
// The decode GEMV applies both while staging its rows / writing its tiles;
// otherwise the standalone kernels run around the plain product.
static int qmm_fused(const uint16_t *x, const uint16_t *res, const uint16_t *nw, float eps, uint16_t *h_out,
                     uint16_t *x_out, const uint32_t *wq, const uint16_t *s, const uint16_t *b, const uint16_t *bias,
                     uint16_t *y, int64_t M, int64_t N, int64_t K, int bits, int group_size, void *stream,
                     int64_t swiglu_half, uint16_t *gu_scratch, const HeadArgmax *head = nullptr,
                     bool *head_done = nullptr) {
    const char *what = swiglu_half ? "qmm_swiglu" : "qmm_rmsnorm";
    const uint16_t *xin = nw ? x_out : x;
    int rc = check_qmm(xin, wq, s, b, y, M, N, K, bits, group_size);
    if (rc) return rc;
    if (!x) return set_error(SC_EINVAL, "%s: null pointer argument", what);
    if (!nw && res) return set_error(SC_EINVAL, "%s: a residual needs the norm weight", what);
    if (K % 8) return set_error(SC_EINVAL, "%s: K=%lld must be a multiple of 8", what, (long long)K);
    if (!aligned(x, 16) || !aligned(res, 16) || !aligned(nw, 16) || !aligned(h_out, 16))
        return set_error(SC_EINVAL, "%s: activation pointers must be 16-byte aligned", what);
    const int64_t n_out = swiglu_half ? swiglu_half : N;
    if (swiglu_half) {
        if (swiglu_half % 8 || N != 2 * swiglu_half)
            return set_error(SC_EINVAL, "%s: the weight must stack gate and up ([2I, K]) with I a multiple of 8", what);
        if (!gu_scratch || !aligned(gu_scratch, 16)) return set_error(SC_EINVAL, "%s: gate_up scratch required", what);
    }
    const size_t xb = (size_t)M * K * 2, yb = (size_t)M * n_out * 2, gb = (size_t)M * N * 2;
    const void *outs[4] = {x_out, h_out, y, gu_scratch};
    const size_t outb[4] = {xb, xb, yb, gb};
    for (int i = 0; i < 4; ++i) {
        if (overlap(outs[i], outb[i], x, xb) || overlap(outs[i], outb[i], res, xb))
            return set_error(SC_EINVAL, "%s: outputs must not overlap the inputs (other workgroups still read them)",
                             what);
        for (int k = 0; k < i; ++k)
            if (overlap(outs[i], outb[i], outs[k], outb[k]))
                return set_error(SC_EINVAL, "%s: output buffers overlap", what);
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (head_done) *head_done = false;
    if (qgemv_dma_eligible(xin, wq, s, b, (int)M, (int)K)) {
        // with a greedy head the batch-1 kernel selects the token itself; where it
        // does not apply the product runs alone and the caller selects
        DmaFused f{nw ? PRO_NORM_KIND : 0, (int)swiglu_half, res, nw, eps, res ? h_out : nullptr, x_out, head};
        rc = launch_qgemv_dma(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, &f);
        if (rc != SC_EUNSUPPORTED) {
            if (head_done) *head_done = head && rc == SC_OK;
            return rc;
        }
        if (head) {
            f.head = nullptr;
            rc = launch_qgemv_dma(x, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, &f);
            if (rc != SC_EUNSUPPORTED) return rc;
        }
    }
    if (nw) {
        rc = launch_rms_norm(x, res, nw, x_out, res ? h_out : nullptr, M, K, eps, st);
        if (rc) return rc;
    }
    if (!swiglu_half) return qmm_dispatch(xin, wq, s, b, bias, y, M, N, K, bits, group_size, stream, SC_QMM_PATH_AUTO);
    if (band_first(M, N, K)) {
        // the band kernel's split-K pass applies silu(gate) * up itself
        rc = launch_qgemm_band(xin, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, false, (int)swiglu_half, 0,
                               0);
        if (rc != SC_EUNSUPPORTED) return rc;
    }
    if (M > 8 && M <= 32) {
        // the 9-32-row GEMV's split-K pass applies silu(gate) * up itself
        rc = launch_qgemv16(xin, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, false, (int)swiglu_half);
        if (rc != SC_EUNSUPPORTED) return rc;
    }
    if (M > 32) {
        // the GEMM pairs gate and up columns in its tiles and writes act itself
        rc = launch_qgemm_mfma(xin, wq, s, b, bias, y, (int)M, (int)N, (int)K, bits, st, (int)swiglu_half);
        if (rc != SC_EUNSUPPORTED) return rc;
    }
    rc = qmm_dispatch(xin, wq, s, b, bias, gu_scratch, M, N, K, bits, group_size, stream, SC_QMM_PATH_AUTO);
    if (rc) return rc;
    return launch_silu_mul(gu_scratch, M, swiglu_half, y, st);
}

}  // namespace sc

using namespace sc;

extern "C" {

int sc_abi_version(void) { return SC_ABI_VERSION; }

const char *sc_last_error(void) { return g_err; }

int sc_qmm_bf16(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                int group_size, void *hip_stream) {
    return qmm_dispatch(x, wq, scales, biases, bias_or_null, y, M, N, K, bits, group_size, hip_stream,
                        SC_QMM_PATH_AUTO);
}

int sc_qmm_bf16_path(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                     const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                     int group_size, int path, void *hip_stream) {
    return qmm_dispatch(x, wq, scales, biases, bias_or_null, y, M, N, K, bits, group_size, hip_stream, path);
}

int sc_qmm_bf16_band(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                     const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                     int group_size, int waves, int ksplit, void *hip_stream) {
    int rc = check_qmm(x, wq, scales, biases, y, M, N, K, bits, group_size);
    if (rc) return rc;
    if (waves != 0 && waves != 4 && waves != 8) return set_error(SC_EINVAL, "qmm_band: waves=%d (0, 4 or 8)", waves);
    if (ksplit < 0 || ksplit > 65535) return set_error(SC_EINVAL, "qmm_band: ksplit=%d", ksplit);
    rc = launch_qgemm_band(x, wq, scales, biases, bias_or_null, y, (int)M, (int)N, (int)K, bits,
                           reinterpret_cast<hipStream_t>(hip_stream), false, 0, waves, ksplit);
    if (rc == SC_EUNSUPPORTED)
        return set_error(SC_EUNSUPPORTED, "qmm_band: M=%lld K=%lld not taken (M <= 256, K %% 512 == 0, 16-byte "
                         "aligned scales and biases)", (long long)M, (long long)K);
    return rc;
}

int sc_qmm_bf16_noalloc(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                        const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                        int group_size, void *hip_stream) {
    return qmm_dispatch(x, wq, scales, biases, bias_or_null, y, M, N, K, bits, group_size, hip_stream,
                        SC_QMM_PATH_AUTO, /*no_alloc=*/true);
}

int sc_vocab_gather_bf16(const void *ids, int ids_is_int64, int64_t T, const uint16_t *table, int64_t v_local,
                         int64_t D, int64_t vocab_start, uint16_t *out, void *hip_stream) {
    if (T < 0 || v_local < 1 || D < 1) return set_error(SC_EINVAL, "vocab_gather: T=%lld v_local=%lld D=%lld",
                                                        (long long)T, (long long)v_local, (long long)D);
    if (T == 0) return SC_OK;
    if (!ids || !table || !out) return set_error(SC_EINVAL, "vocab_gather: null pointer argument");
    if (!aligned(ids, ids_is_int64 ? 8 : 4) || !aligned(table, 2) || !aligned(out, 2))
        return set_error(SC_EINVAL, "vocab_gather: misaligned pointer");
    return launch_vocab_gather(ids, ids_is_int64, T, table, v_local, D, vocab_start, out,
                               reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_qembed_gather_bf16(const void *ids, int ids_is_int64, int64_t T, const uint32_t *wq,
                          const uint16_t *scales, const uint16_t *biases, int64_t v_local, int64_t D,
                          int64_t vocab_start, int bits, int group_size, uint16_t *out, void *hip_stream) {
    if (bits != 4 && bits != 8) return set_error(SC_EUNSUPPORTED, "qembed_gather: bits=%d", bits);
    if (group_size != 64) return set_error(SC_EUNSUPPORTED, "qembed_gather: group_size=%d", group_size);
    if (T < 0 || v_local < 1 || D < 1 || D % 64)
        return set_error(SC_EINVAL, "qembed_gather: T=%lld v_local=%lld D=%lld (D must be a multiple of 64)",
                         (long long)T, (long long)v_local, (long long)D);
    if (T == 0) return SC_OK;
    if (!ids || !wq || !scales || !biases || !out) return set_error(SC_EINVAL, "qembed_gather: null pointer");
    if (!aligned(out, 16) || !aligned(wq, 4)) return set_error(SC_EINVAL, "qembed_gather: misaligned pointer");
    return launch_qembed_gather(ids, ids_is_int64, T, wq, scales, biases, v_local, D, vocab_start, bits, out,
                                reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_dequantize_bf16(const uint32_t *wq, const uint16_t *scales, const uint16_t *biases, int64_t rows,
                       int64_t K, int bits, int group_size, uint16_t *out, void *hip_stream) {
    if (bits != 4 && bits != 8) return set_error(SC_EUNSUPPORTED, "dequantize: bits=%d", bits);
    if (group_size != 64) return set_error(SC_EUNSUPPORTED, "dequantize: group_size=%d", group_size);
    if (rows < 0 || K < 1 || K % 64) return set_error(SC_EINVAL, "dequantize: rows=%lld K=%lld", (long long)rows,
                                                      (long long)K);
    if (rows == 0) return SC_OK;
    if (!wq || !scales || !biases || !out) return set_error(SC_EINVAL, "dequantize: null pointer");
    return launch_dequantize(wq, scales, biases, rows, K, bits, out, reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_quantize_affine(const float *w, int64_t rows, int64_t K, int bits, int group_size, uint32_t *wq,
                       uint16_t *scales, uint16_t *biases, void *hip_stream) {
    if (bits != 4 && bits != 8) return set_error(SC_EUNSUPPORTED, "quantize: bits=%d", bits);
    if (group_size != 64) return set_error(SC_EUNSUPPORTED, "quantize: group_size=%d", group_size);
    if (rows < 0 || K < 1 || K % 64) return set_error(SC_EINVAL, "quantize: rows=%lld K=%lld", (long long)rows,
                                                      (long long)K);
    if (rows == 0) return SC_OK;
    if (!w || !wq || !scales || !biases) return set_error(SC_EINVAL, "quantize: null pointer");
    return launch_quantize(w, rows, K, bits, wq, scales, biases, reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_rms_norm_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *weight, uint16_t *y,
                     uint16_t *h_out_or_null, int64_t rows, int64_t D, float eps, void *hip_stream) {
    return launch_rms_norm(x, residual_or_null, weight, y, h_out_or_null, rows, D, eps,
                           reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_rope_append_kv_bf16(uint16_t *qkv, int64_t qkv_stride, int64_t B, int64_t S, int64_t H, int64_t Hkv,
                           int64_t D, const float *cos_t, const float *sin_t, int64_t table_len, uint16_t *k_cache,
                           uint16_t *v_cache_t, int64_t T_cap, const int32_t *cache_len, int64_t pos_offset,
                           void *hip_stream) {
    return launch_rope_append(qkv, qkv_stride, B, S, H, Hkv, D, cos_t, sin_t, table_len, k_cache, v_cache_t, T_cap,
                              cache_len, pos_offset, reinterpret_cast<hipStream_t>(hip_stream));
}

int64_t sc_attention_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D, int64_t T_cap) {
    return attention_workspace_bytes(B, S, H, Hkv, D, T_cap);
}

int sc_attention_bf16(const uint16_t *q, int64_t q_stride, const uint16_t *k_cache, const uint16_t *v_cache_t,
                      int64_t T_cap, const int32_t *cache_len, uint16_t *out, int64_t out_stride, int64_t B,
                      int64_t S, int64_t H, int64_t Hkv, int64_t D, float scale, void *workspace,
                      int64_t workspace_bytes, void *hip_stream) {
    return launch_attention(q, q_stride, k_cache, v_cache_t, T_cap, cache_len, out, out_stride, B, S, H, Hkv, D,
                            scale, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(hip_stream), nullptr,
                            nullptr);
}

int sc_attention_masked_bf16(const uint16_t *q, int64_t q_stride, const uint16_t *k_cache, const uint16_t *v_cache_t,
                             int64_t T_cap, const int32_t *cache_len, uint16_t *out, int64_t out_stride, int64_t B,
                             int64_t S, int64_t H, int64_t Hkv, int64_t D, float scale, const float *mask,
                             int64_t mask_stride_b, int64_t mask_stride_h, int64_t mask_stride_s,
                             int64_t mask_stride_t, void *workspace, int64_t workspace_bytes, void *hip_stream) {
    if (!mask) return set_error(SC_EINVAL, "attention_masked: null mask");
    const long ms[4] = {mask_stride_b, mask_stride_h, mask_stride_s, mask_stride_t};
    return launch_attention(q, q_stride, k_cache, v_cache_t, T_cap, cache_len, out, out_stride, B, S, H, Hkv, D,
                            scale, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(hip_stream), mask, ms);
}

int64_t sc_attention_decode_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t T_cap) {
    return attention_decode_workspace_bytes(B, H, Hkv, D, T_cap);
}

int sc_attention_decode_bf16(const uint16_t *qkv, int64_t qkv_stride, int64_t B, int64_t H, int64_t Hkv, int64_t D,
                             const float *cos_t, const float *sin_t, int64_t table_len, uint16_t *k_cache,
                             uint16_t *v_cache_t, int64_t T_cap, const int32_t *cache_len, int64_t pos_offset,
                             float scale, uint16_t *out, int64_t out_stride, void *workspace,
                             int64_t workspace_bytes, void *hip_stream) {
    return launch_attention_decode(qkv, qkv_stride, B, H, Hkv, D, cos_t, sin_t, table_len, k_cache, v_cache_t, T_cap,
                                   cache_len, pos_offset, scale, out, out_stride, workspace, workspace_bytes,
                                   reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_attention_decode_masked_bf16(const uint16_t *qkv, int64_t qkv_stride, int64_t B, int64_t H, int64_t Hkv,
                                    int64_t D, const float *cos_t, const float *sin_t, int64_t table_len,
                                    uint16_t *k_cache, uint16_t *v_cache_t, int64_t T_cap, const int32_t *cache_len,
                                    int64_t pos_offset, float scale, const float *mask, int64_t mask_stride_b,
                                    int64_t mask_stride_h, int64_t mask_stride_t, uint16_t *out, int64_t out_stride,
                                    void *workspace, int64_t workspace_bytes, void *hip_stream) {
    if (!mask) return set_error(SC_EINVAL, "attention_decode_masked: null mask");
    const long ms[4] = {(long)mask_stride_b, (long)mask_stride_h, 0, (long)mask_stride_t};
    return launch_attention_decode(qkv, qkv_stride, B, H, Hkv, D, cos_t, sin_t, table_len, k_cache, v_cache_t, T_cap,
                                   cache_len, pos_offset, scale, out, out_stride, workspace, workspace_bytes,
                                   reinterpret_cast<hipStream_t>(hip_stream), mask, ms);
}

int sc_silu_mul_bf16(const uint16_t *gate_up, int64_t rows, int64_t I, uint16_t *out, void *hip_stream) {
    return launch_silu_mul(gate_up, rows, I, out, reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_argmax_bf16(const uint16_t *logits, int64_t rows, int64_t V, int32_t *ids, int32_t *tokens_or_null,
                   int64_t tokens_stride, int64_t tokens_cols, const int32_t *step_or_null, void *hip_stream) {
    return launch_argmax(logits, rows, V, ids, tokens_or_null, tokens_stride, tokens_cols, step_or_null,
                         reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_add_bf16(const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t n, void *hip_stream) {
    return launch_add_bf16(a, b, out, n, reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_add_i32(int32_t *counters, int64_t n, int32_t delta, void *hip_stream) {
    return launch_add_i32(counters, n, delta, reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_decode_plan_create(const sc_decode_model *model, const sc_decode_layer *layers, void **plan_out) {
    return decode_plan_create(model, layers, plan_out);
}

int sc_decode_plan_run(void *plan, void *hip_stream) {
    return decode_plan_run(plan, reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_decode_plan_status(void *plan, uint32_t *status) { return decode_plan_status(plan, status); }

int sc_decode_plan_trace(void *plan, int enable) { return decode_plan_trace(plan, enable); }

int sc_decode_plan_read_trace(void *plan, uint32_t *stamps, int64_t n, int *workgroups, int *ops) {
    return decode_plan_read_trace(plan, stamps, n, workgroups, ops);
}

void sc_decode_plan_destroy(void *plan) { decode_plan_destroy(plan); }

int sc_qmm_rmsnorm_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *norm_weight, float eps,
                        uint16_t *h_out_or_null, uint16_t *xn_out, const uint32_t *wq, const uint16_t *scales,
                        const uint16_t *biases, const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N,
                        int64_t K, int bits, int group_size, void *hip_stream) {
    if (!norm_weight || !xn_out) return set_error(SC_EINVAL, "qmm_rmsnorm: null pointer argument");
    return qmm_fused(x, residual_or_null, norm_weight, eps, h_out_or_null, xn_out, wq, scales, biases, bias_or_null, y,
                     M, N, K, bits, group_size, hip_stream, 0, nullptr);
}

int sc_qmm_add_rmsnorm_bf16(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                            const uint16_t *bias_or_null, const uint16_t *residual, const uint16_t *norm_weight,
                            float eps, uint16_t *h_out, uint16_t *xn_out, int64_t M, int64_t N, int64_t K, int bits,
                            int group_size, void *hip_stream) {
    int rc = check_qmm(x, wq, scales, biases, xn_out, M, N, K, bits, group_size);
    if (rc) return rc;
    if (!residual || !norm_weight || !h_out) return set_error(SC_EINVAL, "qmm_add_rmsnorm: null pointer argument");
    if (N % 8 || N > 16384) return set_error(SC_EINVAL, "qmm_add_rmsnorm: N=%lld must be a multiple of 8 up to 16384",
                                             (long long)N);
    if (!aligned(residual, 16) || !aligned(norm_weight, 16) || !aligned(h_out, 16) || !aligned(xn_out, 16) ||
        !aligned(bias_or_null, 16))
        return set_error(SC_EINVAL, "qmm_add_rmsnorm: activation, weight and bias pointers must be 16-byte aligned");
    const size_t xb = (size_t)M * K * 2, yb = (size_t)M * N * 2;
    if (overlap(h_out, yb, x, xb) || overlap(h_out, yb, residual, yb) || overlap(xn_out, yb, x, xb) ||
        overlap(xn_out, yb, residual, yb) || overlap(h_out, yb, xn_out, yb))
        return set_error(SC_EINVAL, "qmm_add_rmsnorm: h_out and xn_out must not overlap each other or the inputs");
    // the product's split-K partials go straight into the norm's pass; a product that
    // writes its rows itself writes them into xn_out, which the pass then reads
    SplitKeep keep;
    rc = qmm_dispatch(x, wq, scales, biases, bias_or_null, xn_out, M, N, K, bits, group_size, hip_stream,
                      SC_QMM_PATH_AUTO, false, &keep);
    if (rc) return rc;
    return launch_split_add_rms_norm(keep.partials, keep.splits, xn_out, keep.splits ? bias_or_null : nullptr,
                                     residual, norm_weight, h_out, xn_out, M, N, eps,
                                     reinterpret_cast<hipStream_t>(hip_stream));
}

int sc_decode_head_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *norm_weight, float eps,
                        uint16_t *h_out_or_null, uint16_t *xn_out, const uint32_t *wq, const uint16_t *scales,
                        const uint16_t *biases, const uint16_t *bias_or_null, uint16_t *logits, int64_t M, int64_t N,
                        int64_t K, int bits, int group_size, int32_t *ids, int32_t *tokens_or_null,
                        int64_t tokens_stride, int64_t tokens_cols, const int32_t *step_or_null,
                        int32_t *counters_or_null, int64_t n_counters, void *workspace, int64_t workspace_bytes,
                        void *hip_stream) {
    if (!norm_weight || !xn_out || !ids) return set_error(SC_EINVAL, "decode_head: null pointer argument");
    if (n_counters < 0 || n_counters > 64 || (n_counters && !counters_or_null))
        return set_error(SC_EINVAL, "decode_head: n_counters=%lld (at most 64, with a counter buffer)",
                         (long long)n_counters);
    if (!workspace || !aligned(workspace, 16) || workspace_bytes < SC_DECODE_HEAD_WORKSPACE_BYTES)
        return set_error(SC_EINVAL, "decode_head: workspace of %d bytes, 16-byte aligned, required",
                         SC_DECODE_HEAD_WORKSPACE_BYTES);
    if (N < 1 || N > 0x7FFFFFFFLL) return set_error(SC_EINVAL, "decode_head: N=%lld", (long long)N);
    if (tokens_or_null && (tokens_cols < 1 || tokens_stride < tokens_cols))
        return set_error(SC_EINVAL, "decode_head: bad token buffer");
    hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
    HeadArgmax hd{reinterpret_cast<unsigned long long *>(workspace),
                  reinterpret_cast<unsigned *>(static_cast<uint8_t *>(workspace) + 8),
                  ids, tokens_or_null, (long)tokens_cols, step_or_null, counters_or_null, (int)n_counters};
    bool done = false;
    int rc = qmm_fused(x, residual_or_null, norm_weight, eps, h_out_or_null, xn_out, wq, scales, biases, bias_or_null,
                       logits, M, N, K, bits, group_size, hip_stream, 0, nullptr, M == 1 ? &hd : nullptr, &done);
    if (rc || done) return rc;
    rc = launch_argmax(logits, M, N, ids, tokens_or_null, tokens_stride, tokens_cols, step_or_null, st);
    if (rc || !n_counters) return rc;
    return launch_add_i32(counters_or_null, n_counters, 1, st);
}

int sc_qmm_swiglu_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *norm_weight_or_null,
                       float eps, uint16_t *h_out_or_null, uint16_t *xn_out_or_null, const uint32_t *wq,
                       const uint16_t *scales, const uint16_t *biases, const uint16_t *bias_or_null, uint16_t *act_out,
                       uint16_t *gate_up_scratch, int64_t M, int64_t I, int64_t K, int bits, int group_size,
                       void *hip_stream) {
    if (norm_weight_or_null && !xn_out_or_null) return set_error(SC_EINVAL, "qmm_swiglu: xn_out required with a norm");
    return qmm_fused(x, residual_or_null, norm_weight_or_null, eps, h_out_or_null, xn_out_or_null, wq, scales, biases,
                     bias_or_null, act_out, M, 2 * I, K, bits, group_size, hip_stream, I, gate_up_scratch);
}


}  // extern "C"
