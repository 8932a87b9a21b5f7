// Shared device/host helpers for the gfx950 kernels of libshardcompute_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

namespace sc {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// ---------------------------------------------------------------- bf16 bits

__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }

// Round-to-nearest-even fp32 -> bf16 with NaNs kept NaN (quiet bit set).
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f2bf(lo) | (f2bf(hi) << 16);
}

// The same rounding (RNE) in one v_cvt_pk_bf16_f32 for finite values; NaN payloads
// may differ from f2bf, so the bit-compared kernels keep pack_bf16x2.
typedef __bf16 bf16x2_vt __attribute__((ext_vector_type(2)));
typedef float f32x2_vt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    const f32x2_vt v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_vt));
}

// ---------------------------------------------------------------- exact elementwise math
//
// The kernels whose outputs are compared bit for bit (RMSNorm, residual add, SiLU
// gate, RoPE) compute with these: x*y and x+y rounded once each and never fused
// into an FMA (the IR carries no contract flag; HIP's __fmul_rn is a plain
// product that contracts after inlining).  The standalone kernels and the GEMV
// prologues that fuse the same ops share them, so both give identical bits.

__device__ __forceinline__ float mul_rn(float x, float y) {
#pragma clang fp contract(off)
    return x * y;
}
__device__ __forceinline__ float add_rn(float x, float y) {
#pragma clang fp contract(off)
    return x + y;
}

// fp32 value of element e (0..7) of 8 packed bf16
__device__ __forceinline__ float bfe(uint4 v, int e) {
    const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
    return (e & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
}

// ---------------------------------------------------------------- lane exchanges
//
// Butterfly partners on the VALU: DPP moves inside rows of 16 lanes and the gfx950
// permlane swaps across rows, instead of LDS-routed shuffles.  A butterfly step
// v_l + v_(l xor d) gives every lane of a pair the same bits (one rounding of a
// commutative sum), so these reproduce the __shfl_xor trees exactly.

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_XOR1 = 0xB1;          // quad_perm [1, 0, 3, 2]: lane l <- l ^ 1
constexpr int DPP_XOR2 = 0x4E;          // quad_perm [2, 3, 0, 1]: lane l <- l ^ 2
constexpr int DPP_XOR3 = 0x1B;          // quad_perm [3, 2, 1, 0]: lane l <- l ^ 3
constexpr int DPP_HALF_MIRROR = 0x141;  // lane l <- l ^ 7 (within 8)
constexpr int DPP_ROR8 = 0x128;         // lane l <- l ^ 8 (within 16)

// rows of 16 lanes (r0 r1 r2 r3) -> a = (r0 r0 r2 r2), b = (r1 r1 r3 r3)
__device__ __forceinline__ void swap16(float v, float &a, float &b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(p[0]);
    b = __uint_as_float(p[1]);
}
// halves (lo hi) -> a = (lo lo), b = (hi hi)
__device__ __forceinline__ void swap32(float v, float &a, float &b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(p[0]);
    b = __uint_as_float(p[1]);
}
// v + v of lane l ^ 32
__device__ __forceinline__ float xor32_sum(float v) {
    float a, b;
    swap32(v, a, b);
    return a + b;
}
// v of lane l ^ 4
__device__ __forceinline__ float xor4_mov(float v) { return dpp_mov<DPP_HALF_MIRROR>(dpp_mov<DPP_XOR3>(v)); }

// sum over the 8 lanes 8g .. 8g + 7, as the tree over distances 1, 2, 4
__device__ __forceinline__ float group8_sum(float v) {
    v += dpp_mov<DPP_XOR1>(v);
    v += dpp_mov<DPP_XOR2>(v);
    return v + dpp_mov<DPP_HALF_MIRROR>(v);     // after the quad sums, lane l ^ 7 holds lane l ^ 4's value
}

// xor-tree sum over the 64 lanes, distances 32, 16, 8, 4, 2, 1 (every lane gets the
// same total)
__device__ __forceinline__ float wave_sum(float v) {
    float a, b;
    swap32(v, a, b);
    v = a + b;
    swap16(v, a, b);
    v = a + b;
    v += dpp_mov<DPP_ROR8>(v);
    v += xor4_mov(v);
    v += dpp_mov<DPP_XOR2>(v);
    return v + dpp_mov<DPP_XOR1>(v);
}

// bf16(a + b), 8 packed bf16
__device__ __forceinline__ uint4 add_bf16x8(uint4 a, uint4 b) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(add_rn(bfe(a, 2 * e), bfe(b, 2 * e)), add_rn(bfe(a, 2 * e + 1), bfe(b, 2 * e + 1)));
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// ss + h_0^2 + ... + h_7^2, left to right
__device__ __forceinline__ float sumsq_bf16x8(float ss, uint4 v) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float f = bfe(v, e);
        ss = add_rn(ss, mul_rn(f, f));
    }
    return ss;
}

// sqrt(mean + eps) from the row's sum of squares (transformer.py:52)
__device__ __forceinline__ float rms_root(float tot, int D, float eps) {
    return __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)D), eps));
}

// h / root, correctly rounded, with one division per row instead of one per element:
// y = RN(1 / root) (the caller's), q = RN(h y), then RN(q + r y) with the remainder
// r = h - q root, exact in one fma.  With y within half an ulp of 1 / root and q within
// one ulp of h / root this is the correctly rounded quotient (Markstein's correction
// step), barring overflow and underflow; root is a positive RMS and the quotients of
// bf16 activations are normal.
__device__ __forceinline__ float div_root(float h, float root, float y) {
    const float q = mul_rn(h, y);
    return fmaf(fmaf(-q, root, h), y, q);
}

// bf16((h / root) * w): divide by the root, then scale (transformer.py:55).  Every
// kernel that normalises (standalone, the GEMV prologues, the decode trunk) uses this,
// so they agree bit for bit; the rounding is RNE in one instruction per pair (a NaN
// input stays NaN, its payload may differ from f2bf's)
__device__ __forceinline__ uint4 norm_bf16x8(uint4 h, uint4 w, float root) {
    const float y = __fdiv_rn(1.f, root);        // loop-invariant where the row's root is
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o[e] = cvt_pk_bf16(mul_rn(div_root(bfe(h, 2 * e), root, y), bfe(w, 2 * e)),
                           mul_rn(div_root(bfe(h, 2 * e + 1), root, y), bfe(w, 2 * e + 1)));
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// (g / (1 + exp(-g))) * u in fp32 (parallel/mlp.py:161-162, 244)
__device__ __forceinline__ float silu_mul_f(float g, float u) {
    return mul_rn(__fdiv_rn(g, add_rn(1.f, expf(-g))), u);
}

// bf16(silu(g) * u), 8 packed bf16
__device__ __forceinline__ uint4 silu_mul_bf16x8(uint4 g, uint4 u) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(silu_mul_f(bfe(g, 2 * e), bfe(u, 2 * e)), silu_mul_f(bfe(g, 2 * e + 1), bfe(u, 2 * e + 1)));
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// Row RMS partition shared by every kernel that normalises a row: 256 threads,
// thread t sums chunks t, t + 256, ... (8 elements each, in order), then each
// wave reduces with wave_sum and the 4 wave partials are added in order.
constexpr int NORM_THREADS = 256;

// ---------------------------------------------------------------- MLX affine codes
//
// W4: one uint32 word holds codes q0..q7 of 8 consecutive k, q_j in bits [4j, 4j+4).
// nib_pair(w, 4r) is the bf16 pair (128 + q_r, 128 + q_{r+4}): OR-ing a code into
// the mantissa of 128.0 (0x4300) gives 128 + q exactly.  The 4 pairs of a word
// are MFMA operand slots [q0 q4 q1 q5 q2 q6 q3 q7].
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int shift) {
    return ((w >> shift) & 0x000F000Fu) | 0x43004300u;
}

// Slot order of nib_pair for one word: slot s holds code k_of_slot(s) of the word.
__host__ __device__ constexpr int w4_slot_k(int s) { return (s >> 1) + 4 * (s & 1); }

// W8: one word holds 4 byte codes q0..q3.  Codes up to 255 need 8 significant
// bits, which bf16 holds exactly: convert through fp32 and keep the top half.
// (float)(byte) lowers to a single v_cvt_f32_ubyteN.
__device__ __forceinline__ float ubyte_f32(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFFu); }
__device__ __forceinline__ uint32_t byte_pair_lo(uint32_t w) {
    return __builtin_amdgcn_perm(__float_as_uint(ubyte_f32(w, 1)), __float_as_uint(ubyte_f32(w, 0)), 0x07060302u);
}
__device__ __forceinline__ uint32_t byte_pair_hi(uint32_t w) {
    return __builtin_amdgcn_perm(__float_as_uint(ubyte_f32(w, 3)), __float_as_uint(ubyte_f32(w, 2)), 0x07060302u);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    uint4 v = make_uint4(a, b, c, d);
    return __builtin_bit_cast(bf16x8_t, v);
}
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace sc

// ---------------------------------------------------------------- host side

namespace sc {

// Sets the thread-local message returned by sc_last_error(); returns `code`.
int set_error(int code, const char *fmt, ...);

enum Status {
    SC_OK = 0,
    SC_EINVAL = -1,      // bad argument (shape, pointer, bits, group size)
    SC_EUNSUPPORTED = -2,
    SC_ELAUNCH = -3,     // HIP runtime error
};

struct DeviceInfo {
    int num_cus = 0;
    int max_lds_per_block = 0;
};
const DeviceInfo &device_info();

// Library-owned per-device split-K scratch (partials + arrival counters).
struct SplitKScratch {
    float *partials = nullptr;
    unsigned *counters = nullptr;
};
int splitk_scratch(size_t partial_floats, size_t n_counters, SplitKScratch *out);

// The allocation-free entry point's split-K partials: this device's file-scope
// array of SC_QMM_NOALLOC_SCRATCH_BYTES (address looked up once per device).
int qmm_noalloc_scratch(float **out);

// A split-K product whose caller runs its own pass over the fp32 partials
// [splits, M, N] instead of launch_qmm_finalize; splits = 0 when the product wrote y
// itself (one split).
struct SplitKeep {
    const float *partials = nullptr;
    int splits = 0;
};

// y = bf16(sum over splits of partials [splits, M, N] in split order) (+ bias after
// rounding); with half > 0 the product is gate|up stacked (N = 2 half) and y [M, half]
// receives silu(gate) * up of the rounded values.
int launch_qmm_finalize(const float *partials, int splits, int M, int N, const uint16_t *bias, uint16_t *y, int half,
                        hipStream_t stream);

// Arg-max key of a bf16 value: the order-preserving 16-bit image of the value
// (NaN above +inf, -0.0 equal to +0.0) over ~index, so the larger key is the larger
// value and, among equal values, the smaller index.  No key is 0.
__device__ __forceinline__ unsigned long long argmax_key(uint32_t u, uint32_t idx) {
    u &= 0xFFFFu;
    uint32_t k;
    if ((u & 0x7FFFu) > 0x7F80u) k = 0xFFFFu;
    else {
        if (u == 0x8000u) u = 0;
        k = (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
    }
    return ((unsigned long long)k << 32) | (0xFFFFFFFFu - idx);
}

// Greedy token selection folded into a batch-1 GEMV's epilogue: every workgroup
// maxes the keys of its outputs into *key; the last one to finish (counted in
// *done) writes ids[0] and tokens[step[0]] (when 0 <= step[0] < tok_cols), adds 1
// to counters[0, n_counters), and leaves *key and *done zero for the next call.
struct HeadArgmax {
    unsigned long long *key;
    unsigned *done;
    int32_t *ids;
    int32_t *tokens;
    long tok_cols;
    const int32_t *step;
    int32_t *counters;
    int n_counters;
};

// Input transformation a decode GEMV can apply while staging its rows (see
// qgemv_dma.hip): 1 = RMSNorm of x (+ res), 2 = silu(gate) * up of x = gate|up.
struct DmaFused {
    int kind;
    int swiglu_half;     // > 0: paired gate|up tiles, output act [M, swiglu_half]
    const uint16_t *res;
    const uint16_t *norm_weight;
    float eps;
    uint16_t *h_out;
    uint16_t *x_out;
    const HeadArgmax *head = nullptr;   // batch-1 plain-output GEMV only
};

}  // namespace sc

#define SC_HIP_CHECK(expr)                                                               \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return ::sc::set_error(::sc::SC_ELAUNCH, "%s failed: %s", #expr,              \
                                   hipGetErrorString(e_));                               \
    } while (0)
