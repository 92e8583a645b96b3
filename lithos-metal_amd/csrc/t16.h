// The T16 weight pack and the M = 1 GEMV building blocks shared by the GEMV kernels (gemv.hip) and the fused GEMV
// chain (chain.hip): formats, tile / chunk / scale-piece offsets, the exact NVFP4 decode helpers, the gated head norm
// and the fixed-order sums over a tile's K slices.
#pragma once
#include "mi_common.h"

namespace {

constexpr int FMT_NVFP4 = MI_FMT_NVFP4;
constexpr int FMT_INT4 = MI_FMT_INT4_AFFINE;
constexpr int FMT_BF16 = MI_FMT_BF16;
constexpr int FMT_FP8 = MI_FMT_FP8_E4M3;

constexpr int UNIT_Q = 1152;   // int4 unit: 1024 B codes + 128 B (scale, bias) pairs
constexpr int UNIT_B = 1024;   // bf16 unit: 16 rows × 32 columns
constexpr int GROUP_REC = 18;  // grouped-mode record: expert, count, 16 pair ids

__host__ __device__ constexpr int unit_bytes(int fmt) { return fmt == FMT_BF16 || fmt == FMT_FP8 ? UNIT_B : UNIT_Q; }
__host__ __device__ constexpr int chunk_cols(int fmt) { return fmt == FMT_BF16 ? 32 : fmt == FMT_FP8 ? 64 : 128; }

// NVFP4 tile layout: groups of 8 chunks, each [g × 1 KiB codes][scale block: 64 pieces of 16 B (8 B if g <= 4)]
__host__ __device__ inline int nv_group_chunks(int gi, int chunks) { return min(8, chunks - 8 * gi); }
__host__ __device__ inline int nv_piece(int g) { return g > 4 ? 16 : 8; }
__host__ __device__ inline long long nv_tile_bytes(int chunks) {
  const int r = chunks & 7;
  return (long long)(chunks >> 3) * 9216 + (r ? r * 1024 + 64 * nv_piece(r) : 0);
}
__host__ __device__ inline long long nv_code_off(int c) { return (long long)(c >> 3) * 9216 + (c & 7) * 1024; }
__host__ __device__ inline long long nv_scale_off(int gi, int chunks) {
  return (long long)gi * 9216 + nv_group_chunks(gi, chunks) * 1024;
}
__host__ __device__ inline long long tile_bytes(int fmt, int chunks) {
  return fmt == FMT_NVFP4 ? nv_tile_bytes(chunks) : (long long)chunks * unit_bytes(fmt);
}

// The mantissa factor ±1.mmm of a decoded E4M3 block scale (FP32 bits u; every nonzero E4M3 value, subnormals
// included, is an FP32 normal), or ±0 for a zero scale: the power-of-two part is then 0.0, which the scaled FP4
// conversions read as 2^-127 — BF16 keeps that, so the block must be zeroed by its factor
__device__ __forceinline__ float nv_mant(uint32_t u) {
  return __uint_as_float((u & 0x7F800000u) ? ((u & 0x807FFFFFu) | 0x3F800000u) : (u & 0x80000000u));
}

// byte j of dw (two E2M1 codes, low nibble first) → BF16 pair × 2^E (exact); j is a compile-time constant after
// unrolling, as the instruction's byte select requires
__device__ __forceinline__ bf16x2 cvt_fp4x2_bf16(uint32_t dw, float e, int j) {
  switch (j) {
    case 0: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(dw, e, 0);
    case 1: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(dw, e, 1);
    case 2: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(dw, e, 2);
    default: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(dw, e, 3);
  }
}

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + __expf(-v)); }

// the Gated DeltaNet output norm (nn/gdn.py:86-93, the gdn_norm op) on one lane's 8 consecutive input values at
// `col` of token row `xrow`, whose 128-column head spans this lane's 16-lane row (every lane of the wave calls it):
// x ← bf16(bf16(bf16(w)·bf16(x·r))·silu(z)), r = rsqrt(mean over the head of x² + eps)
__device__ __forceinline__ void gated_head_norm8(uint32_t (&qq)[4], const uint4 zv, const float4 w0, const float4 w1,
                                                 float eps) {
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = bf16_bits_to_f32(qq[i] & 0xFFFFu), hi = bf16_bits_to_f32(qq[i] >> 16);
    sq = fmaf(lo, lo, fmaf(hi, hi, sq));
  }
  const float r = 1.0f / sqrtf(sum16(sq) / 128.0f + eps);
  const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  const uint32_t zz[4] = {zv.x, zv.y, zv.z, zv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float x = bf16_bits_to_f32(h ? qq[i] >> 16 : qq[i] & 0xFFFFu);
      const float z = bf16_bits_to_f32(h ? zz[i] >> 16 : zz[i] & 0xFFFFu);
      const float nw = round_bf16(round_bf16(wv[2 * i + h]) * round_bf16(x * r));
      o[h] = nw * silu_f(z);
    }
    qq[i] = (uint32_t)f32_to_bf16_bits(o[0]) | ((uint32_t)f32_to_bf16_bits(o[1]) << 16);
  }
}

// orders this wave's LDS writes before its later LDS reads by other lanes (one wave's LDS requests complete in
// order; this keeps the compiler from moving them)
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); __builtin_amdgcn_wave_barrier(); }

// Σ over the S K slices of one tile row in the order every M = 1 kernel uses: four partial sums p_q over slices
// q, q + 4, … (q = 0..3) in increasing order, then (p0 + p1) + (p2 + p3). slice_sum runs it on a whole wave — lane
// (r = l % 16, q = l / 16) forms p_q of row r and the rows meet through two lane exchanges — and returns the row's
// total in every lane; slice_sum_lane is the same sum in one lane.
__device__ __forceinline__ float slice_sum(const float* red, int stride, int S, int lane) {
  const int r = lane & 15, q = lane >> 4;
  float v = 0.0f;
  for (int w = q; w < S; w += 4) v += red[w * stride + r];
  return add_xor32(add_xor16(v));
}
__device__ __forceinline__ float slice_sum_lane(const float* red, int stride, int S, int r) {
  float p[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    p[q] = 0.0f;
    for (int w = q; w < S; w += 4) p[q] += red[w * stride + r];
  }
  return (p[0] + p[1]) + (p[2] + p[3]);
}

}  // namespace
