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

// The library's own scratch buffers (split-K partials and fold counters, attention partials, argmax counters) for
// callers that pass none: one per (kind, device, stream), so calls on different streams never share one. A buffer is
// zeroed when allocated (kernels that keep counters leave them at zero). It grows on demand but is never freed
// before the process ends — a graph captured earlier keeps the address it recorded — and it refuses to grow while
// the stream is being captured (the caller runs one eager call of the shape first, or passes its own workspace).
enum MiScratchKind { MI_SCRATCH_GEMV = 0, MI_SCRATCH_GQA = 1, MI_SCRATCH_ARGMAX = 2, MI_SCRATCH_CHAIN = 3 };
int mi_library_scratch(int kind, size_t bytes, hipStream_t stream, void** out);

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
// A workgroup barrier that orders LDS only: the waves' outstanding global loads (the next chunks in flight) stay in
// flight across it, where __syncthreads' release would first wait for every one of them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t u16) { return __uint_as_float(u16 << 16); }

// round-to-nearest-even, NaN kept quiet (the reference's f32_to_bf16): gfx950's v_cvt_pk_bf16_f32, branch-free
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float round_bf16(float f) { return (float)(__bf16)f; }

// ---- wave64 cross-lane exchanges without LDS: DPP inside a row of 16 lanes, gfx950's permlane16/32 swaps across
// rows. They read every lane of the wave: call them with the whole wave active. ---------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i of 8 ↔ 7 − i
constexpr int kDppMirror = 0x140;      // lane i of 16 ↔ 15 − i

// sum / max over the 16 lanes of a row, result in every lane of the row
__device__ __forceinline__ float sum16(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return v;
}
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return v;
}

// v(l) + v(l ^ 16) and v(l) + v(l ^ 32): a swap leaves each lane holding its own value in one half of the pair and
// its partner's in the other, so the pair's sum (max) is the same in both lanes
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

// sum over the four lanes l, l^16, l^32, l^48 (the k-groups of an MFMA operand)
__device__ __forceinline__ float quad16_sum(float v) { return add_xor32(add_xor16(v)); }

__device__ __forceinline__ float wave_sum(float v) { return quad16_sum(sum16(v)); }
__device__ __forceinline__ float wave_max(float v) { return max_xor32(max_xor16(max16(v))); }
