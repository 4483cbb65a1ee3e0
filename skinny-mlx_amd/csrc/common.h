// Internal helpers shared by the HIP translation units of libskinny_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "skinny_hip.h"

// Records a formatted message for skinny_last_error() and returns `code`.
int skinny_set_error(int code, const char* fmt, ...);

#define SKINNY_CHECK_ARG(cond, ...)                          \
  do {                                                       \
    if (!(cond)) return skinny_set_error(SKINNY_EINVAL, __VA_ARGS__); \
  } while (0)

// Checks the launch that was just enqueued; returns SKINNY_ELAUNCH with the HIP
// error string on failure.
int skinny_check_launch(const char* what);

__host__ __device__ static inline bool skinny_aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Index of the calling wave in its workgroup, as a value the compiler knows to be uniform across
// the wave (threadIdx.x >> 6 is, but divergence analysis cannot prove it): anything derived from
// it can live in SGPRs, e.g. buffer-load soffsets, which otherwise become per-load waterfall loops.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// fp32 -> bf16 bits, round to nearest even: gfx950's v_cvt_pk_bf16_f32 (one instruction, where
// the integer rounding sequence took five or six).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// silu(z) = z / (1 + e^-z) from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; about
// 1 ulp each, far below the bf16 rounding that follows): the Gated-DeltaNet output norm's gate,
// shared by every kernel that forms that norm so that all of them produce the same bits. At
// z -> -inf the sum overflows to inf and the gate is -0, at z -> +inf it is z.
__device__ __forceinline__ float silu_gate(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -1.44269504f));
}

// SwiGLU of one element pair, from bf16 gate and up values: silu(g) * u in fp32, rounded to bf16.
// Shared by the standalone activation kernel and the fused gate|up matmul epilogue so that both
// paths produce the same bits.
__device__ __forceinline__ uint16_t silu_mul_bf16(float g, float u) {
  return f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
}

// Row sums by DPP moves: xor 1 and xor 2 inside quads (quad_perm), then the mirror inside 8 lanes
// and inside 16 (row_half_mirror, row_mirror) pair the same partial sums as xor 4 and xor 8 would,
// so every lane of a 16-lane row gets the xor butterfly's sum, bit for bit, at VALU latency
// instead of an LDS-crossbar round trip per step.
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_add<0xB1>(v);      // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);      // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);     // row_half_mirror
  return dpp_add<0x140>(v);  // row_mirror
}

// Sum over the 64 lanes of a wave, the same in every lane: row sums, then (r0 + r1) + (r2 + r3)
// of the four rows through v_readlane.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0)), r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32)), r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}
