// Helpers shared by the LDS-DMA decode GEMVs (qgemv_dma.hip, qgemv_m1.hip): the
// item ring geometry, the global_load_lds issue and the vmcnt / lgkmcnt waits that
// pace it, and the small operand transforms of the W4 / W8 codes.
#pragma once
#include "sc_common.h"

namespace sc {
namespace dma {

// An "item" is 16 weight rows x 256 contiguous bytes (4 KB) plus the 16 rows'
// scales and biases for those bytes' groups (1 KB slot tail).
constexpr int RING = 3;                     // items per wave ring (RING-1 in flight)
constexpr int DMA_PER_ITEM = 5;             // 4 weight + 1 scale/bias instruction
constexpr int SLOT_W = 4096;                // weight bytes per item
constexpr int SLOT_BYTES = SLOT_W + 1024;   // + scales (lanes 0-15) and biases (16-31)
constexpr int S2_UNITS = SLOT_W / 1024 + 1; // 1 KB staging units in one ring slot

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f4;

__device__ __forceinline__ uint32_t wc(uint4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
__device__ __forceinline__ uint32_t wh(uint4 v, int i) {
    const uint32_t w = wc(v, i >> 1);
    return (i & 1) ? (w >> 16) : (w & 0xFFFFu);
}

__device__ __forceinline__ uint4 perm_w4x(uint4 v) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    return o;
}

// 16 bytes per active lane from global `g` to LDS byte address lds_base + 16 * lane.
// The instruction takes its LDS base from M0, which this block sets itself; the
// kernel has no other M0 user (no LDS-DMA builtins, no indirect register access),
// so declaring the clobber is all the compiler needs (it warns regardless).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base))
                 : "memory", "m0");
}
// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit byte offset per
// lane (the SADDR form: no 64-bit address per lane in VGPRs).
__device__ __forceinline__ void dma16s(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds_base))
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// (x & mask) | magic.  VOP3 on gfx950 takes no literal and one scalar operand, so
// with both constants as literals the compiler emits and + or; with the mask in an
// SGPR and the magic in a VGPR (both opaque to constant folding) it selects one
// v_and_or_b32 and still tracks the VALU-write -> MFMA-read hazard itself, which it
// would not do for the same instruction written as inline asm.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask_sgpr, uint32_t magic_vgpr) {
    return (x & mask_sgpr) | magic_vgpr;
}

__device__ __forceinline__ void wait_lgkm0() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most n vector-memory operations of this wave are outstanding
// (lgkmcnt / expcnt untouched).
template <int n>
__device__ __forceinline__ void wait_vm() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace dma
}  // namespace sc
