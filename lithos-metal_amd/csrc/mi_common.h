// Shared device/host helpers for the gfx950 decode-layer kernels: BF16/F16 bit conversions, wave64 reductions,
// the error plumbing of the C ABI (every entry point returns 0 or an MI_E* code; mi_last_error() has the text).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/lithos_mi355.h"

typedef _Float16 f16_t;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---- host-side error state --------------------------------------------------------------------------------------
int mi_set_error(int code, const char* fmt, ...);          // records the message, returns code
int mi_check_hip(hipError_t e, const char* what);         // 0 on success, else MI_E_HIP with the HIP message

#define MI_TRY_HIP(expr, what)                          \
  do {                                                  \
    int _rc = mi_check_hip((expr), (what));             \
    if (_rc) return _rc;                                \
  } while (0)

#define MI_REQUIRE(cond, ...)                                        \
  do {                                                               \
    if (!(cond)) return mi_set_error(MI_E_INVALID, __VA_ARGS__);      \
  } while (0)

// ---- BF16 / F16 bit helpers ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t u16) { return __uint_as_float(u16 << 16); }

// round-to-nearest-even, NaN kept quiet (the reference's f32_to_bf16)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---- wave64 reductions (DPP/permute via the compiler's cross-lane builtins) ----------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// sum over the four lanes l, l^16, l^32, l^48 (the k-groups of an MFMA operand)
__device__ __forceinline__ float quad16_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}
