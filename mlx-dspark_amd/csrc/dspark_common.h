// Shared helpers for the gfx950 kernels: vector types, bf16 conversions, the MFMA wrapper,
// and the host-side status/error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dspark.h"

namespace dspark {

using u16 = uint16_t;
using u32 = uint32_t;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef u32 u32x4_t __attribute__((ext_vector_type(4)));
typedef u32 u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- device helpers

__device__ __forceinline__ float bf2f(u32 bits16) { return __builtin_bit_cast(float, bits16 << 16); }

__device__ __forceinline__ u16 f2bf(float f) {
  // round-to-nearest-even (v_cvt_pk_bf16_f32)
  return __builtin_bit_cast(u16, (__bf16)f);
}

// SwiGLU of bf16 gate and up values as mlx rounds it: bf16(bf16(g * bf16(sigmoid(g))) * u)
// (the caller rounds the returned product)
__device__ __forceinline__ float swiglu_bf16(float g, float u) {
  const float sg = bf2f(f2bf(1.0f / (1.0f + expf(-g))));
  return bf2f(f2bf(g * sg)) * u;
}

__device__ __forceinline__ u32 pack_bf16x2(float lo, float hi) {
  bf16x2_t p = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(u32, p);
}

// D = A(16 x 32) * B(32 x 16) + C, bf16 operands, fp32 accumulate.
// Operand layout (wave64): lane l supplies row/column (l & 15) and the 8 reduction slots
// 8*(l >> 4) .. +7; any consistent assignment of reduction indices to (l >> 4, element)
// across A and B gives the same sum. Output: lane l holds D[4*(l >> 4) + r][l & 15], r = 0..3.
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4_t ldg128(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x2_t ldg64(const void* p) {
  return *reinterpret_cast<const u32x2_t*>(p);
}
// Streamed-once data (weights, K/V tiles): the non-temporal hint ("nt") marks the lines for
// early eviction, so a stream that is read once does not push reused lines out of L2 / MALL.
// A read-only probe of 108 MB in one launch streams 6.4 TB/s with it and 6.1 TB/s without.
__device__ __forceinline__ u32x4_t ldg128_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ u32x2_t ldg64_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
}

// Wave64 cross-lane exchange (ds_bpermute, no LDS storage).
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  const int lane = __lane_id();
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, v)));
}

// max(v, v of lane l ^ 16) and max(v, v of lane l ^ 32) in every lane, with the gfx950 row
// swaps (v_permlane16_swap: rows 0 <-> 1 and 2 <-> 3 of 16 lanes; v_permlane32_swap: the two
// 32-lane halves) on two copies of v: after the swap each lane holds its own value in one
// register and its partner's in the other, in an order that depends on the lane, which a
// commutative max does not see (the same bits as a ds_bpermute exchange, without its LDS
// round trip). Inline asm: given the same value twice, the builtins' two results are folded
// into one by the compiler (they differ: the swap moves rows). s_nop 1 covers the wait states
// between a VALU write of either register and the swap reading it.
__device__ __forceinline__ float max_xor16(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}

// Sum over each aligned group of 8 lanes, returned to all 8: the butterfly over lane bits 0,
// 1, 2 (v + v^1, then + v^2, then + v^4) with DPP exchanges (quad permutes, half-row mirror:
// lane i of an 8-lane group pairs with 7 - i, which holds the other quad's sum).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float sum8_lanes(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm 1,0,3,2
  v += dpp_mov<0x4E>(v);   // quad_perm 2,3,0,1
  v += dpp_mov<0x141>(v);  // row_half_mirror
  return v;
}

// (v & m) | o. Written in C, not as inline asm, so the compiler sees the VALU write: an MFMA
// that reads the result needs two wait states after it, which the compiler inserts only for
// instructions it can see (an inline-asm v_and_or_b32 feeding the unpacked weights to an MFMA
// one instruction later gave wrong products in some schedules). It selects one v_and_or_b32
// when m sits in an SGPR and o in a VGPR (opaque_sgpr / opaque_vgpr); with both as literals it
// would emit a v_and and a v_or.
__device__ __forceinline__ u32 and_or(u32 v, u32 m, u32 o) { return (v & m) | o; }

// A constant the compiler must keep in a scalar / vector register instead of folding it into
// the instructions that use it (an empty asm: no instruction, so nothing is hidden from the
// hazard tracking; identical ones are shared).
__device__ __forceinline__ u32 opaque_sgpr(u32 v) {
  asm("" : "+s"(v));
  return v;
}
__device__ __forceinline__ u32 opaque_vgpr(u32 v) {
  asm("" : "+v"(v));
  return v;
}

// Wave-uniform copy of a value the compiler cannot prove uniform (e.g. threadIdx.x >> 6).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------- host helpers

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Turns a failed launch into DSPARK_ERR_LAUNCH with the HIP error text.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace dspark
