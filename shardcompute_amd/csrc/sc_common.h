// Shared device/host helpers for the gfx950 kernels of libshardcompute_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

}  // namespace sc

#define SC_HIP_CHECK(expr)                                                               \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return ::sc::set_error(::sc::SC_ELAUNCH, "%s failed: %s", #expr,              \
                                   hipGetErrorString(e_));                               \
    } while (0)
