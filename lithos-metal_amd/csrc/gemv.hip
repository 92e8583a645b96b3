// GEMV / skinny GEMM over the T16 weight pack, for M = 1 decode and M ≤ 16 verify, dense or grouped by expert.
//
// Semantics (ops/gemv.py:1-12, nn/linear.py:114-135, kernels/common/gemv_T.metal:232-587): y[t][n] = Σ_k x[t][k]·W[n][k]
// with FP32 accumulation and one BF16 rounding, optional RMSNorm on the input (norm_apply fused on load,
// ops/norm.py:1-6) and a residual / silu·mul epilogue. Grouped mode is the MoE expert GEMV (ops/moe.py `moe_gemv`):
// a group is one expert with the ≤ 16 (token, slot) pairs routed to it, so a step streams exactly the chosen experts.
//
// MI355X design:
//  * One wave64 owns RT 16-row tiles over a run of 128-column chunks. Each chunk of a tile is one 1152-byte unit: a
//    fully coalesced 1 KiB load of 16-byte code words (lane l: row l%16, 32 codes) plus 128 B of block scales.
//  * The products run on MFMA v_mfma_f32_16x16x32_{f16,bf16} with A = activations (16 token rows, padded with an LDS
//    zero row) and B = decoded weights. NVFP4 decodes to exact F16: v_cvt_scalef32_pk_f16_fp4 applies the power-of-two
//    part of the E4M3 block scale, a packed F16 multiply its 3-bit mantissa (e2m1·e4m3 has ≤ 6 significant bits and
//    lies in [2^-10, 2688], so every decoded weight is exact). INT4 codes become exact F16 integers (0x6400|c − 1024)
//    and the affine term is applied per group of 64 as scale·Σcx + bias·Σx.
//  * F16 activations: each token row staged in LDS is multiplied by a power of two 2^-P that brings its max into
//    [2^14, 2^15), converted BF16 → F16 (exact above 2^-14, i.e. everything within 2^28 of the row max), and the
//    partial sums are multiplied back by 2^P — BF16 range without F16 overflow.
//  * Each wave keeps 8/RT chunks of loads in flight (a register ring), issued before the activations are staged, so
//    the staging prologue and the LDS barriers hide under HBM traffic.
//  * K is split across the waves of a workgroup (reduced through LDS in a fixed order, deterministic). When the
//    staged activations of the whole K would not fit LDS (M = 8 over K = 17408), the workgroup walks K in windows,
//    restaging per window. There is no cross-workgroup reduction: on gfx950 the agent-scope fences it needs
//    (an L2 writeback + invalidate per workgroup) cost more than the GEMV.
#include "mi_common.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace {

constexpr int FMT_NVFP4 = MI_FMT_NVFP4;
constexpr int FMT_INT4 = MI_FMT_INT4_AFFINE;
constexpr int FMT_BF16 = MI_FMT_BF16;

constexpr int UNIT_Q = 1152;   // nvfp4 / int4 unit: 1024 B codes + 128 B scales
constexpr int UNIT_B = 1024;   // bf16 unit: 16 rows × 32 columns
constexpr int GROUP_REC = 18;  // grouped-mode record: expert, count, 16 pair ids

__host__ __device__ constexpr int unit_bytes(int fmt) { return fmt == FMT_BF16 ? UNIT_B : UNIT_Q; }
__host__ __device__ constexpr int chunk_cols(int fmt) { return fmt == FMT_BF16 ? 32 : 128; }

struct Args {
  const uint8_t* w;
  const float* row_scale;
  const uint16_t* x;
  uint16_t* y;
  const uint16_t* res;
  const float* norm_w;
  const int32_t* groups;
  long long expert_stride;  // bytes between experts' packs
  float eps;
  int ldx, ldy, ldr;
  int n, k, m;
  int n_tiles, chunks, row_blocks;
  int kw, win, wave_lds;    // chunks per wave (its K slice), chunks per staged window, LDS bytes per wave
  int epilogue, top_k, x_per_slot, out_f32;
  int lds_rows, lds_ld;     // staged token rows, LDS row stride (elements)
};

// ---- weight decode ---------------------------------------------------------------------------------------------
// E4M3 block-scale byte pair → (power-of-two parts, signed mantissa factors as F16)
struct ScalePair {
  float e0, e1;
  f16_t m0, m1;
};

__device__ __forceinline__ ScalePair nvfp4_scales(uint32_t two_bytes) {
  f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)two_bytes, false);   // OCP E4M3 → exact FP32
  uint32_t u0 = __float_as_uint(f.x), u1 = __float_as_uint(f.y);
  ScalePair s;
  s.e0 = __uint_as_float(u0 & 0x7F800000u);
  s.e1 = __uint_as_float(u1 & 0x7F800000u);
  s.m0 = (f16_t)__uint_as_float((u0 & 0x807FFFFFu) | 0x3F800000u);   // ±1.mmm, exact in F16
  s.m1 = (f16_t)__uint_as_float((u1 & 0x807FFFFFu) | 0x3F800000u);
  return s;
}

// 8 E2M1 codes (one dword, low nibble first) → 8 exact F16 weights × block scale (without the tensor scale)
__device__ __forceinline__ f16x8 nvfp4_decode8(uint32_t dw, float e, f16_t mant) {
  const f16x2 mm = {mant, mant};
  f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, e, 0) * mm;
  f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, e, 1) * mm;
  f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, e, 2) * mm;
  f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, e, 3) * mm;
  return f16x8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}

// 8 unsigned nibbles → exact F16 codes in the order (n0, n4, n1, n5, n2, n6, n3, n7); the staged activations use
// the same order inside each group of 8 columns
__device__ __forceinline__ f16x8 int4_decode8(uint32_t dw) {
  const f16x2 off = {(f16_t)1024.0f, (f16_t)1024.0f};
  union { uint32_t u; f16x2 h; } p0, p1, p2, p3;
  p0.u = (dw & 0x000F000Fu) | 0x64006400u;
  p1.u = ((dw >> 4) & 0x000F000Fu) | 0x64006400u;
  p2.u = ((dw >> 8) & 0x000F000Fu) | 0x64006400u;
  p3.u = ((dw >> 12) & 0x000F000Fu) | 0x64006400u;
  f16x2 h0 = p0.h - off, h1 = p1.h - off, h2 = p2.h - off, h3 = p3.h - off;
  return f16x8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
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

__device__ __forceinline__ int int4_perm8(int i) { return (i & 1) ? 4 + (i >> 1) : (i >> 1); }

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + __expf(-v)); }

__device__ __forceinline__ void store_out(const Args& a, long long idx, float v) {
  if (a.out_f32) reinterpret_cast<float*>(a.y)[idx] = v;
  else a.y[idx] = f32_to_bf16_bits(v);
}


// one output value: row tile·16 + m_row of token t, already scaled by its row scale; `up` is the value of the row
// 8 below it (the up half of a silu·mul tile), fetched by the caller with a shuffle every lane executes
__device__ __forceinline__ void emit(const Args& a, const int32_t* pairs, int cnt, int tile, bool tile_ok, int m_row,
                                     int t, float v, float up) {
  if (!tile_ok || t >= cnt) return;
  const int yr = pairs ? pairs[t] : t;
  if (a.epilogue == MI_EPI_SILU_MUL || a.epilogue == MI_EPI_SILU_MUL_ROUNDED) {
    const int col = tile * 8 + m_row;
    if (m_row >= 8 || col >= a.n / 2) return;
    float o;
    if (a.epilogue == MI_EPI_SILU_MUL_ROUNDED) {
      const float gb = round_bf16(v), ub = round_bf16(up);
      o = silu_f(gb) * ub;
    } else {
      o = silu_f(v) * up;
    }
    store_out(a, (long long)yr * a.ldy + col, o);
  } else {
    const int row = tile * 16 + m_row;
    if (row >= a.n) return;
    float o = v;
    if (a.epilogue == MI_EPI_RESIDUAL) o += bf16_bits_to_f32(a.res[(long long)t * a.ldr + row]);
    store_out(a, (long long)yr * a.ldy + row, o);
  }
}

// ---- the kernel ------------------------------------------------------------------------------------------------
template <int FMT>
struct Units {               // one chunk of one tile, in registers
  uint4 q;
  uint32_t s;                // nvfp4: two E4M3 block-scale bytes
  uint2 sb;                  // int4: (scale, bias) pairs of the chunk's two groups
};

template <int FMT>
__device__ __forceinline__ void load_unit(Units<FMT>& u, const uint8_t* p, int lane) {
  u.q = *reinterpret_cast<const uint4*>(p + 16 * lane);
  if constexpr (FMT == FMT_NVFP4) u.s = *reinterpret_cast<const uint16_t*>(p + 1024 + 2 * lane);
  if constexpr (FMT == FMT_INT4) u.sb = *reinterpret_cast<const uint2*>(p + 1024 + 8 * (lane & 15));
}

// orders this wave's LDS writes before its later LDS reads by other lanes (one wave's LDS requests complete in
// order; this keeps the compiler from moving them)
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); __builtin_amdgcn_wave_barrier(); }

// Per-wave LDS region (2-byte elements): xs[lds_rows][lds_ld] staged activations of the wave's current window,
// then pscale[16], and (int4) gsum[win/64][16]. After the regions: stat[waves][16] (fused-norm partial sums).
template <int FMT, int RT>
__global__ __launch_bounds__(512) void gemv_t16(Args a) {
  constexpr int D = 8 / RT;                      // prefetch depth in chunks
  constexpr int KC = chunk_cols(FMT);
  constexpr int UB = unit_bytes(FMT);
  constexpr int XV = 4;                          // activation vectors per lane loaded ahead of the weights
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int rb = blockIdx.x;
  const int grp = blockIdx.y;

  // ---- group: which matrix and which token rows ---------------------------------------------------------------
  int expert = 0, cnt = a.m;
  const int32_t* pairs = nullptr;
  if (a.groups) {
    const int32_t* g = a.groups + grp * GROUP_REC;
    expert = g[0];
    cnt = g[1];
    pairs = g + 2;
    if (cnt <= 0 || expert < 0) return;      // the whole workgroup leaves together: no barrier is skipped
  }
  if (cnt > a.lds_rows) cnt = a.lds_rows;
  auto xrow_of = [&](int j) -> long long {     // activation row of token j (grouped mode: the pair's row)
    if (!pairs) return j;
    const int p = pairs[j];
    return a.x_per_slot ? p : p / a.top_k;
  };

  // ---- this wave: K slice [c0, c0 + kw) chunks, windows of `win` chunks --------------------------------------
  const int c0 = wave * a.kw;
  const int win = a.win;                      // chunks per window
  const int wcols = win * KC;
  uint8_t* wbase_lds = smem + (size_t)wave * a.wave_lds;
  uint16_t* xs = reinterpret_cast<uint16_t*>(wbase_lds);
  float* pscale = reinterpret_cast<float*>(wbase_lds + (size_t)a.lds_rows * a.lds_ld * 2);   // [16] 2^p
  float* pinv = pscale + 16;                                                                  // [16] 2^-p
  float* rstd = pinv + 16;                                                                    // [16]
  float* gsum = rstd + 16;                                                                    // [win·KC/64][16]
  float* stat = reinterpret_cast<float*>(smem + (size_t)nwaves * a.wave_lds);   // [nwaves][16]
  const uint8_t* zero = reinterpret_cast<const uint8_t*>(stat + nwaves * 16); // 64 zero bytes
  if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(stat + nwaves * 16)[threadIdx.x] = 0u;
  if (lane < 16) { rstd[lane] = 1.0f; pscale[lane] = 1.0f; pinv[lane] = 1.0f; }

  const int tile0 = rb * RT;
  bool tile_ok[RT];
  const uint8_t* tbase[RT];
  const uint8_t* wmat = a.w + (long long)expert * a.expert_stride;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    tile_ok[r] = (tile0 + r) < a.n_tiles;
    tbase[r] = wmat + (long long)(tile_ok[r] ? tile0 + r : 0) * a.chunks * UB;
  }

  // activations of window w: cnt rows × wcols columns from column (c0 + w·win)·KC (clamped at the row end)
  uint4 xv[XV];
  auto x_issue = [&](int w) {
    const int per_row = wcols / 8;
    const int n_units = cnt * per_row;
    const int kbase = (c0 + w * win) * KC;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int idx = min(lane + 64 * i, n_units - 1);
      const int j = idx / per_row, e = (idx - j * per_row) * 8;
      const int col = min(kbase + e, a.k - 8);
      xv[i] = *reinterpret_cast<const uint4*>(a.x + xrow_of(j) * a.ldx + col);
    }
  };

  // ---- weights: the first D chunks of every tile --------------------------------------------------------------
  x_issue(0);
  Units<FMT> ring[D][RT];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int c = c0 + min(i, a.kw - 1);
#pragma unroll
    for (int r = 0; r < RT; ++r) load_unit<FMT>(ring[i][r], tbase[r] + (long long)c * UB, lane);
  }

  // ---- fused RMSNorm: Σh² over the row from every wave's slice, one workgroup barrier -------------------------
  if (a.norm_w) {
    const int per_row = a.kw * KC / 8;
    for (int j = 0; j < cnt; ++j) {
      float s = 0.0f;
      for (int u = lane; u < per_row; u += 64) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.x + xrow_of(j) * a.ldx + c0 * KC + u * 8);
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bf16_bits_to_f32(vv[q] & 0xFFFFu), hi = bf16_bits_to_f32(vv[q] >> 16);
          s = fmaf(lo, lo, fmaf(hi, hi, s));
        }
      }
      s = wave_sum(s);
      if (lane == 0) stat[wave * 16 + j] = s;
    }
    __syncthreads();
    if (lane < cnt) {
      float s = 0.0f;
      for (int wv = 0; wv < nwaves; ++wv) s += stat[wv * 16 + lane];          // fixed order: bit-repeatable
      rstd[lane] = 1.0f / sqrtf(s / (float)a.k + a.eps);
    }
    wave_lds_sync();
  }

  // ---- stage window w of this wave's slice into its LDS region (wave-local: no workgroup barrier) -------------
  // x = bf16(h·r·w) when the norm is fused; for F16 operands a per-token power of two 2^-p taken from this window's
  // max brings the row into [2^14, 2^15) before BF16 → F16 (exact from 2^-14 up); the window's products are scaled
  // back by 2^p when folded into the accumulator.
  auto stage = [&](int w) {
    const int per_row = wcols / 8;
    const int n_units = cnt * per_row;
    const int kbase = (c0 + w * win) * KC;
    auto put = [&](int idx, uint4 v) {
      const int j = idx / per_row, e = (idx - j * per_row) * 8;
      const int col = kbase + e;
      if (col >= a.k) {
        v = uint4{0u, 0u, 0u, 0u};                                   // window past the row end
      } else if (a.norm_w) {
        const float4 w0 = *reinterpret_cast<const float4*>(a.norm_w + col);
        const float4 w1 = *reinterpret_cast<const float4*>(a.norm_w + col + 4);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        const float rr = rstd[j];
        uint32_t* vv = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = round_bf16((bf16_bits_to_f32(vv[q] & 0xFFFFu) * rr) * wv[2 * q]);
          const float hi = round_bf16((bf16_bits_to_f32(vv[q] >> 16) * rr) * wv[2 * q + 1]);
          vv[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
        }
      }
      *reinterpret_cast<uint4*>(xs + (size_t)j * a.lds_ld + e) = v;
    };
#pragma unroll
    for (int i = 0; i < XV; ++i)
      if (lane + 64 * i < n_units) put(lane + 64 * i, xv[i]);
    for (int idx = lane + 64 * XV; idx < n_units; idx += 64) {
      const int j = idx / per_row, e = (idx - j * per_row) * 8;
      const int col = min(kbase + e, a.k - 8);
      put(idx, *reinterpret_cast<const uint4*>(a.x + xrow_of(j) * a.ldx + col));
    }
    wave_lds_sync();
    if constexpr (FMT == FMT_BF16) return;
    // per-token prescale from the staged window
    for (int j = 0; j < cnt; ++j) {
      float m = 0.0f;
      for (int u = lane; u < per_row; u += 64) {
        const uint4 v = *reinterpret_cast<const uint4*>(xs + (size_t)j * a.lds_ld + u * 8);
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) m = fmaxf(m, fmaxf(fabsf(bf16_bits_to_f32(vv[q] & 0xFFFFu)), fabsf(bf16_bits_to_f32(vv[q] >> 16))));
      }
      m = wave_max(m);
      if (lane == 0) {
        const int p = (m == 0.0f) ? 0 : (int)((__float_as_uint(m) >> 23) & 0xFF) - 127 - 14;
        pscale[j] = __uint_as_float((uint32_t)(127 + p) << 23);   // 2^p
        pinv[j] = __uint_as_float((uint32_t)(127 - p) << 23);     // 2^-p
      }
    }
    wave_lds_sync();
    for (int idx = lane; idx < n_units; idx += 64) {
      const int j = idx / per_row, e = (idx - j * per_row) * 8;
      uint16_t* p = xs + (size_t)j * a.lds_ld + e;
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      const uint16_t* hv = reinterpret_cast<const uint16_t*>(&v);
      const float sc = pinv[j];
      f16x8 o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (f16_t)(bf16_bits_to_f32(hv[(FMT == FMT_INT4) ? int4_perm8(i) : i]) * sc);
      *reinterpret_cast<f16x8*>(p) = o;
    }
    wave_lds_sync();
    if constexpr (FMT == FMT_INT4) {
      const int ng = wcols / 64;
      for (int idx = lane; idx < 16 * ng; idx += 64) {
        const int g = idx >> 4, j = idx & 15;
        float sum = 0.0f;
        if (j < cnt) {
          const f16_t* p = reinterpret_cast<const f16_t*>(xs + (size_t)j * a.lds_ld + g * 64);
          for (int i = 0; i < 64; ++i) sum += (float)p[i];
        }
        gsum[g * 16 + j] = sum;
      }
      wave_lds_sync();
    }
  };

  const int g4 = lane >> 4;        // k-group of the operands / token quad of the result
  const int m_row = lane & 15;     // A row = token
  const bool a_real = m_row < cnt;
  const uint8_t* a_row = a_real ? reinterpret_cast<const uint8_t*>(xs + (size_t)m_row * a.lds_ld) : zero;
  const int a_mask = a_real ? ~0 : 0;    // a padding token reads the same 16 zero bytes at every step

  // one chunk of RT tiles on MFMA, the activations of window-local column kl
  auto compute = [&](const Units<FMT>* u, int kl, f32x4* acc) {
    if constexpr (FMT == FMT_BF16) {
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(a_row + (((kl + 8 * g4) * 2) & a_mask));
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        union { uint4 u; bf16x8 b; } wv;
        wv.u = u[r].q;
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, wv.b, acc[r], 0, 0, 0);
      }
    } else if constexpr (FMT == FMT_NVFP4) {
      f16x8 av[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) av[s] = *reinterpret_cast<const f16x8*>(a_row + (((kl + 32 * g4 + 8 * s) * 2) & a_mask));
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const ScalePair sp = nvfp4_scales(u[r].s);
        const uint32_t dw[4] = {u[r].q.x, u[r].q.y, u[r].q.z, u[r].q.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const f16x8 bv = nvfp4_decode8(dw[s], s < 2 ? sp.e0 : sp.e1, s < 2 ? sp.m0 : sp.m1);
          acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[s], bv, acc[r], 0, 0, 0);
        }
      }
    } else {  // INT4: steps 0,1 = group 2c, steps 2,3 = group 2c+1
      f16x8 av[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) av[s] = *reinterpret_cast<const f16x8*>(a_row + (((kl + 32 * s + 8 * g4) * 2) & a_mask));
      const int gl = kl / 64;
      const f32x4 sxa = *reinterpret_cast<const f32x4*>(gsum + gl * 16 + 4 * g4);
      const f32x4 sxb = *reinterpret_cast<const f32x4*>(gsum + (gl + 1) * 16 + 4 * g4);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const uint32_t dw[4] = {u[r].q.x, u[r].q.y, u[r].q.z, u[r].q.w};
        f32x4 da = {0.f, 0.f, 0.f, 0.f}, db = {0.f, 0.f, 0.f, 0.f};
        da = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[0], int4_decode8(dw[0]), da, 0, 0, 0);
        da = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[1], int4_decode8(dw[1]), da, 0, 0, 0);
        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[2], int4_decode8(dw[2]), db, 0, 0, 0);
        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[3], int4_decode8(dw[3]), db, 0, 0, 0);
        const float sca = bf16_bits_to_f32(u[r].sb.x & 0xFFFFu), bia = bf16_bits_to_f32(u[r].sb.x >> 16);
        const float scb = bf16_bits_to_f32(u[r].sb.y & 0xFFFFu), bib = bf16_bits_to_f32(u[r].sb.y >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r][i] = fmaf(sca, da[i], fmaf(bia, sxa[i], acc[r][i]));
          acc[r][i] = fmaf(scb, db[i], fmaf(bib, sxb[i], acc[r][i]));
        }
      }
    }
  };

  // ---- main loop: the wave's K slice window by window, D chunks of every tile in flight -------------------------
  f32x4 acc[RT], wacc[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) { acc[r] = f32x4{0.f, 0.f, 0.f, 0.f}; wacc[r] = acc[r]; }
  auto fold = [&]() {                          // acc += window accumulator · 2^p (per token)
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[r][i] = fmaf(wacc[r][i], pscale[4 * g4 + i], acc[r][i]);
        wacc[r][i] = 0.0f;
      }
  };
  stage(0);
  for (int base = 0; base < a.kw; base += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int cc = base + i;
      if (cc < a.kw) {
        const int w = cc / win, cw = cc - w * win;
        if (cw == 0 && w > 0) {                 // next window of this wave's slice (multi-window plans only)
          fold();
          x_issue(w);
          stage(w);
        }
        compute(ring[i], cw * KC, wacc);
      }
      const int c = c0 + min(cc + D, a.kw - 1);
#pragma unroll
      for (int r = 0; r < RT; ++r) load_unit<FMT>(ring[i][r], tbase[r] + (long long)c * UB, lane);
    }
  }
  fold();

  // ---- reduce the K-slices through LDS, in wave order ------------------------------------------------------------
  if (nwaves > 1) {
    f32x4* red = reinterpret_cast<f32x4*>(smem);     // aliases the staged activations: all reads are done
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RT; ++r) red[(wave * RT + r) * 64 + lane] = acc[r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      f32x4 s = red[r * 64 + lane];
      for (int w = 1; w < nwaves; ++w) {
        const f32x4 o = red[(w * RT + r) * 64 + lane];
        s[0] += o[0]; s[1] += o[1]; s[2] += o[2]; s[3] += o[3];
      }
      acc[r] = s;
    }
  }


  // ---- epilogue ------------------------------------------------------------------------------------------------
  const int n_pad = a.n_tiles * 16;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int row = (tile0 + r) * 16 + m_row;
    const float rs = (a.row_scale != nullptr) ? a.row_scale[(long long)expert * n_pad + (tile_ok[r] ? row : 0)] : 1.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = acc[r][i] * rs;
      const float up = __shfl_down(v, 8, 16);                     // rows 8..15 of a silu·mul tile are the up rows
      emit(a, pairs, cnt, tile0 + r, tile_ok[r], m_row, 4 * g4 + i, v, up);
    }
  }
}

// ---- the M ≤ 2 kernel: VALU dot products on BF16 activations ---------------------------------------------------
// At one or two tokens the MFMA tile would be 15/16 padding and the activations would need the F16 staging; here
// the weights decode to BF16 (v_cvt_scalef32_pk_bf16_fp4: e2m1·2^E exactly), v_dot2_f32_bf16 multiplies them with
// the BF16 activations as they are, and each E4M3 block's 3-bit mantissa factor is applied once per block of 16.
// INT4 codes become BF16 128 + c (0x4300|c, exact) and the dot product is corrected by 128·Σx per 16-column
// segment; the affine pair is applied as scale·Σcx + bias·Σx. Lane (r = l%16, g = l/16) owns row r of each tile
// and 32 of each chunk's 128 columns; the four g-lanes of a row are summed at the end.
template <int FMT, int RT, int MT>
__global__ __launch_bounds__(512) void gemv_dot(Args a) {
  constexpr int D = 8 / RT;
  constexpr int KC = chunk_cols(FMT);
  constexpr int UB = unit_bytes(FMT);
  constexpr int XV = 4;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int rb = blockIdx.x;
  const int grp = blockIdx.y;
  int expert = 0, cnt = a.m;
  const int32_t* pairs = nullptr;
  if (a.groups) {
    const int32_t* g = a.groups + grp * GROUP_REC;
    expert = g[0];
    cnt = g[1];
    pairs = g + 2;
    if (cnt <= 0 || expert < 0) return;
  }
  if (cnt > MT) cnt = MT;
  auto xrow_of = [&](int j) -> long long {
    if (!pairs) return j;
    const int p = pairs[j];
    return a.x_per_slot ? p : p / a.top_k;
  };
  // this wave's K slice: chunks [c0, c1) (slices differ by at most one chunk)
  const int c0 = (int)((long long)wave * a.chunks / nwaves);
  const int c1 = (int)((long long)(wave + 1) * a.chunks / nwaves);
  const int kw = c1 - c0;
  const int scols = kw * KC;
  // LDS per wave: xs[MT][slice cols] BF16 (INT4: permuted in 8s) | (INT4) seg[MT][kw][2][4] Σx per 16-col segment
  uint8_t* wl = smem + (size_t)wave * a.wave_lds;
  uint16_t* xs = reinterpret_cast<uint16_t*>(wl);
  const int ld = a.lds_ld;
  float* seg = reinterpret_cast<float*>(wl + (size_t)MT * ld * 2);
  float* stat = reinterpret_cast<float*>(smem + (size_t)nwaves * a.wave_lds);   // [nwaves][16]
  float* red = stat + nwaves * 16;                                             // [nwaves][RT][MT][16]

  const int tile0 = rb * RT;
  bool tile_ok[RT];
  const uint8_t* tbase[RT];
  const uint8_t* wmat = a.w + (long long)expert * a.expert_stride;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    tile_ok[r] = (tile0 + r) < a.n_tiles;
    tbase[r] = wmat + (long long)(tile_ok[r] ? tile0 + r : 0) * a.chunks * UB;
  }

  // activation slice loads first, then the weight ring: the wait for the activations counts the weights behind them
  const int per_row = scols / 8;
  const int n_units = cnt * per_row;
  uint4 xv[XV];
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int idx = min(lane + 64 * i, n_units - 1);
    const int j = idx / per_row, e = (idx - j * per_row) * 8;
    xv[i] = *reinterpret_cast<const uint4*>(a.x + xrow_of(j) * a.ldx + c0 * KC + e);
  }
  Units<FMT> ring[D][RT];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int c = c0 + min(i, kw - 1);
#pragma unroll
    for (int r = 0; r < RT; ++r) load_unit<FMT>(ring[i][r], tbase[r] + (long long)c * UB, lane);
  }

  // fused RMSNorm statistic over the full row: per-wave partial sums, one barrier, fixed summation order
  float rstd0 = 1.0f, rstd1 = 1.0f;
  if (a.norm_w) {
    for (int j = 0; j < cnt; ++j) {
      float s = 0.0f;
      for (int u = lane; u < per_row; u += 64) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.x + xrow_of(j) * a.ldx + c0 * KC + u * 8);
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bf16_bits_to_f32(vv[q] & 0xFFFFu), hi = bf16_bits_to_f32(vv[q] >> 16);
          s = fmaf(lo, lo, fmaf(hi, hi, s));
        }
      }
      s = wave_sum(s);
      if (lane == 0) stat[wave * 16 + j] = s;
    }
    __syncthreads();
    float s0 = 0.0f, s1 = 0.0f;
    for (int wv = 0; wv < nwaves; ++wv) { s0 += stat[wv * 16]; if (MT > 1) s1 += stat[wv * 16 + 1]; }
    rstd0 = 1.0f / sqrtf(s0 / (float)a.k + a.eps);
    rstd1 = 1.0f / sqrtf(s1 / (float)a.k + a.eps);
  }

  // stage the slice (BF16; normalized when fused; INT4: the (0,4,1,5,2,6,3,7) order inside each 8)
  auto put = [&](int idx, uint4 v) {
    const int j = idx / per_row, e = (idx - j * per_row) * 8;
    uint32_t* vv = reinterpret_cast<uint32_t*>(&v);
    if (a.norm_w) {
      const int col = c0 * KC + e;
      const float4 w0 = *reinterpret_cast<const float4*>(a.norm_w + col);
      const float4 w1 = *reinterpret_cast<const float4*>(a.norm_w + col + 4);
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      const float rr = j == 0 ? rstd0 : rstd1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = round_bf16((bf16_bits_to_f32(vv[q] & 0xFFFFu) * rr) * wv[2 * q]);
        const float hi = round_bf16((bf16_bits_to_f32(vv[q] >> 16) * rr) * wv[2 * q + 1]);
        vv[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
      }
    }
    if constexpr (FMT == FMT_INT4) {        // (x0,x1)(x2,x3)(x4,x5)(x6,x7) → (x0,x4)(x1,x5)(x2,x6)(x3,x7)
      const uint32_t a0 = vv[0], a1 = vv[1], a2 = vv[2], a3 = vv[3];
      vv[0] = __builtin_amdgcn_perm(a2, a0, 0x05040100u);
      vv[1] = __builtin_amdgcn_perm(a2, a0, 0x07060302u);
      vv[2] = __builtin_amdgcn_perm(a3, a1, 0x05040100u);
      vv[3] = __builtin_amdgcn_perm(a3, a1, 0x07060302u);
    }
    *reinterpret_cast<uint4*>(xs + (size_t)j * ld + e) = v;
  };
#pragma unroll
  for (int i = 0; i < XV; ++i)
    if (lane + 64 * i < n_units) put(lane + 64 * i, xv[i]);
  for (int idx = lane + 64 * XV; idx < n_units; idx += 64) {
    const int j = idx / per_row, e = (idx - j * per_row) * 8;
    put(idx, *reinterpret_cast<const uint4*>(a.x + xrow_of(j) * a.ldx + c0 * KC + e));
  }
  wave_lds_sync();
  if constexpr (FMT == FMT_INT4) {
    // Σx over each (chunk, g, group) segment of 16 columns: steps {0,1} (group A) / {2,3} (group B) of k-group g
    const int nseg = MT * kw * 8;
    for (int idx = lane; idx < nseg; idx += 64) {
      const int j = idx / (kw * 8), rem = idx - j * kw * 8;
      const int cc = rem >> 3, g = (rem >> 1) & 3, gp = rem & 1;
      float s = 0.0f;
      if (j < cnt) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const uint4 v = *reinterpret_cast<const uint4*>(xs + (size_t)j * ld + cc * 128 + 32 * (2 * gp + st) + 8 * g);
          const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) s += bf16_bits_to_f32(vv[q] & 0xFFFFu) + bf16_bits_to_f32(vv[q] >> 16);
        }
      }
      seg[idx] = s;
    }
    wave_lds_sync();
  }

  const int g = lane >> 4, m_row = lane & 15;
  float acc[RT][MT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = 0.0f;

  auto compute = [&](const Units<FMT>* u, int cc) {
    if constexpr (FMT == FMT_NVFP4) {
      uint4 xq[MT][4];                          // this lane's 32 activations of the chunk, per token
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * g + 8 * s);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)u[r].s, false);
        const uint32_t u0 = __float_as_uint(f.x), u1 = __float_as_uint(f.y);
        const float e[2] = {__uint_as_float(u0 & 0x7F800000u), __uint_as_float(u1 & 0x7F800000u)};
        const float mant[2] = {__uint_as_float((u0 & 0x807FFFFFu) | 0x3F800000u),
                               __uint_as_float((u1 & 0x807FFFFFu) | 0x3F800000u)};
        const uint32_t dw[4] = {u[r].q.x, u[r].q.y, u[r].q.z, u[r].q.w};
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          float part[MT];
#pragma unroll
          for (int t = 0; t < MT; ++t) part[t] = 0.0f;
#pragma unroll
          for (int s = 2 * b; s < 2 * b + 2; ++s) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const bf16x2 w2 = cvt_fp4x2_bf16(dw[s], e[b], j);
#pragma unroll
              for (int t = 0; t < MT; ++t) {
                const uint32_t xw = j == 0 ? xq[t][s].x : j == 1 ? xq[t][s].y : j == 2 ? xq[t][s].z : xq[t][s].w;
                part[t] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf16x2, xw), part[t], false);
              }
            }
          }
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[r][t] = fmaf(part[t], mant[b], acc[r][t]);
        }
      }
    } else if constexpr (FMT == FMT_INT4) {
      uint4 xq[MT][4];
      float sa[MT], sb[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * s + 8 * g);
        sa[t] = seg[(t * kw + cc) * 8 + g * 2];
        sb[t] = seg[(t * kw + cc) * 8 + g * 2 + 1];
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const uint32_t dw[4] = {u[r].q.x, u[r].q.y, u[r].q.z, u[r].q.w};
        float d[2][MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) d[0][t] = d[1][t] = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t w2 = ((dw[s] >> (4 * j)) & 0x000F000Fu) | 0x43004300u;   // BF16 (128 + n_j, 128 + n_j+4)
#pragma unroll
            for (int t = 0; t < MT; ++t) {
              const uint32_t xw = j == 0 ? xq[t][s].x : j == 1 ? xq[t][s].y : j == 2 ? xq[t][s].z : xq[t][s].w;
              d[s >> 1][t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w2), __builtin_bit_cast(bf16x2, xw),
                                                             d[s >> 1][t], false);
            }
          }
        }
        const float sca = bf16_bits_to_f32(u[r].sb.x & 0xFFFFu), bia = bf16_bits_to_f32(u[r].sb.x >> 16);
        const float scb = bf16_bits_to_f32(u[r].sb.y & 0xFFFFu), bib = bf16_bits_to_f32(u[r].sb.y >> 16);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[r][t] = fmaf(sca, fmaf(-128.0f, sa[t], d[0][t]), fmaf(bia, sa[t], acc[r][t]));
          acc[r][t] = fmaf(scb, fmaf(-128.0f, sb[t], d[1][t]), fmaf(bib, sb[t], acc[r][t]));
        }
      }
    } else {  // BF16 weights: 8 values of row r at columns 32·cc + 8·g
      uint4 xq[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) xq[t] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 32 + 8 * g);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const uint32_t dw[4] = {u[r].q.x, u[r].q.y, u[r].q.z, u[r].q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const uint32_t xw = j == 0 ? xq[t].x : j == 1 ? xq[t].y : j == 2 ? xq[t].z : xq[t].w;
            acc[r][t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, dw[j]), __builtin_bit_cast(bf16x2, xw),
                                                         acc[r][t], false);
          }
      }
    }
  };

  for (int base = 0; base < kw; base += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int cc = base + i;
      if (cc < kw) compute(ring[i], cc);
      const int c = c0 + min(cc + D, kw - 1);
#pragma unroll
      for (int r = 0; r < RT; ++r) load_unit<FMT>(ring[i][r], tbase[r] + (long long)c * UB, lane);
    }
  }

  // the four k-groups of each row, then the K-slices (waves) in order
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = quad16_sum(acc[r][t]);
  if (nwaves > 1) {
    if (g == 0) {
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[((wave * RT + r) * MT + t) * 16 + m_row] = acc[r][t];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        float s = red[((0 * RT + r) * MT + t) * 16 + m_row];
        for (int w = 1; w < nwaves; ++w) s += red[((w * RT + r) * MT + t) * 16 + m_row];
        acc[r][t] = s;
      }
  }
  const int n_pad = a.n_tiles * 16;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int row = (tile0 + r) * 16 + m_row;
    const float rs = (a.row_scale != nullptr) ? a.row_scale[(long long)expert * n_pad + (tile_ok[r] ? row : 0)] : 1.0f;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float v = acc[r][t] * rs;
      const float up = __shfl_down(v, 8, 16);
      if (g == 0) emit(a, pairs, cnt, tile0 + r, tile_ok[r], m_row, t, v, up);
    }
  }
}

// ---- exact dequantization through the same decode ---------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(64) void dequant_t16(const uint8_t* w, const float* row_scale, int n, int k, int chunks,
                                                   float* out) {
  const int lane = threadIdx.x;
  const int tile = blockIdx.x / chunks, c = blockIdx.x % chunks;
  constexpr int UB = unit_bytes(FMT);
  const uint8_t* u = w + ((long long)tile * chunks + c) * UB;
  const uint4 q = *reinterpret_cast<const uint4*>(u + 16 * lane);
  const int row = tile * 16 + (lane & 15), g = lane >> 4;
  if (row >= n) return;
  float* o = out + (long long)row * k;
  const uint32_t dw[4] = {q.x, q.y, q.z, q.w};
  if constexpr (FMT == FMT_NVFP4) {
    const ScalePair sp = nvfp4_scales(*reinterpret_cast<const uint16_t*>(u + 1024 + 2 * lane));
    const float rs = row_scale ? row_scale[row] : 1.0f;
    for (int s = 0; s < 4; ++s) {
      const f16x8 v = nvfp4_decode8(dw[s], s < 2 ? sp.e0 : sp.e1, s < 2 ? sp.m0 : sp.m1);
      for (int i = 0; i < 8; ++i) o[c * 128 + 32 * g + 8 * s + i] = (float)v[i] * rs;
    }
  } else if constexpr (FMT == FMT_INT4) {
    const uint2 sb = *reinterpret_cast<const uint2*>(u + 1024 + 8 * (lane & 15));
    for (int s = 0; s < 4; ++s) {
      const f16x8 v = int4_decode8(dw[s]);
      const uint32_t pr = s < 2 ? sb.x : sb.y;
      const float sc = bf16_bits_to_f32(pr & 0xFFFFu), bi = bf16_bits_to_f32(pr >> 16);
      for (int i = 0; i < 8; ++i) o[c * 128 + 32 * s + 8 * g + int4_perm8(i)] = fmaf((float)v[i], sc, bi);
    }
  } else {
    for (int i = 0; i < 8; ++i) {
      const uint32_t h = (dw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      o[c * 32 + 8 * g + i] = bf16_bits_to_f32(h);
    }
  }
}

// ---- planning --------------------------------------------------------------------------------------------------
struct Plan {
  int dot;                 // 1: the VALU kernel (M <= 2), 0: MFMA
  int rt, wk, kw, win;
  int lds_rows, lds_ld, wave_lds;
  size_t lds_bytes;
};

int check_desc(const mi_gemv_desc* d) {
  MI_REQUIRE(d, "mi_gemv: null descriptor");
  MI_REQUIRE(d->format == FMT_NVFP4 || d->format == FMT_INT4 || d->format == FMT_BF16, "mi_gemv: unknown format %d",
             d->format);
  const int kc = chunk_cols(d->format);
  MI_REQUIRE(d->n > 0 && d->k > 0 && d->k % kc == 0, "mi_gemv: k=%d must be a positive multiple of %d", d->k, kc);
  MI_REQUIRE(d->m >= 1 && (d->groups || d->m <= 16), "mi_gemv: dense mode needs 1 <= m <= 16 (m=%d)", d->m);
  MI_REQUIRE(d->w && d->x && d->y, "mi_gemv: null weight, input or output pointer");
  MI_REQUIRE(d->ldx >= d->k, "mi_gemv: ldx=%d < k=%d", d->ldx, d->k);
  MI_REQUIRE(d->epilogue >= MI_EPI_NONE && d->epilogue <= MI_EPI_SILU_MUL_ROUNDED, "mi_gemv: bad epilogue");
  MI_REQUIRE(d->epilogue != MI_EPI_RESIDUAL || d->residual, "mi_gemv: residual epilogue without residual");
  const bool silu = d->epilogue == MI_EPI_SILU_MUL || d->epilogue == MI_EPI_SILU_MUL_ROUNDED;
  MI_REQUIRE(!silu || d->n % 16 == 0, "mi_gemv: silu_mul needs n %% 16 == 0 (8 gate + 8 up rows per tile)");
  MI_REQUIRE(d->ldy >= (silu ? d->n / 2 : d->n), "mi_gemv: ldy too small");
  MI_REQUIRE(!d->groups || (d->max_groups > 0 && d->top_k > 0), "mi_gemv: grouped mode needs max_groups and top_k");
  MI_REQUIRE(((uintptr_t)d->x & 15) == 0 && d->ldx % 8 == 0, "mi_gemv: x must be 16-byte aligned with ldx %% 8 == 0");
  MI_REQUIRE(((uintptr_t)d->w & 15) == 0, "mi_gemv: weight pack must be 16-byte aligned");
  MI_REQUIRE(!d->norm_w || ((uintptr_t)d->norm_w & 15) == 0, "mi_gemv: norm_w must be 16-byte aligned");
  return MI_OK;
}

constexpr size_t kLdsBudget = 64 * 1024;

size_t wave_lds_for(int fmt, int rows, int win_cols) {
  size_t b = (size_t)rows * (win_cols + 8) * 2 + 3 * 16 * 4 + (fmt == FMT_INT4 ? (size_t)(win_cols / 64) * 16 * 4 : 0);
  return (b + 15) / 16 * 16;
}

Plan make_plan(const mi_gemv_desc* d) {
  const int fmt = d->format;
  int force[3] = {0, 0, 0};   // MI_GEMV_PLAN="rt,wk,win" pins a plan (tuning sweeps)
  if (const char* env = getenv("MI_GEMV_PLAN")) sscanf(env, "%d,%d,%d", &force[0], &force[1], &force[2]);
  const int kc = chunk_cols(fmt);
  const int chunks = d->k / kc;
  const int n_tiles = (d->n + 15) / 16;
  const int groups = d->groups ? d->max_groups : 1;
  const int rows = d->groups ? std::min(16, d->m) : d->m;   // a group holds at most one pair per token
  Plan best{};
  double best_score = -1e30;
  const char* fk = getenv("MI_GEMV_KERNEL");                 // "dot" / "mfma" pins the kernel (tuning sweeps)
  const bool dot_ok = rows <= 2 && !(fk && fk[0] == 'm');
  if (dot_ok) {
    for (int rt : {1, 2, 4}) {
      if (force[0] && rt != force[0]) continue;
      for (int wk = 1; wk <= 8; ++wk) {
        if (force[0] && wk != force[1]) continue;
        const int kwmax = (chunks + wk - 1) / wk;
        if (kwmax < 1 || chunks < wk) continue;
        size_t wl = (size_t)rows * (kwmax * kc + 8) * 2 + (fmt == FMT_INT4 ? (size_t)rows * kwmax * 8 * 4 : 0);
        wl = (wl + 15) / 16 * 16;
        const size_t lds = (size_t)wk * wl + (size_t)wk * 16 * 4 + (size_t)wk * rt * rows * 16 * 4;
        if (lds > kLdsBudget) continue;
        const int row_blocks = (n_tiles + rt - 1) / rt;
        const double wgs = (double)row_blocks * groups;
        const double waves = wgs * wk;
        const int per_cu = std::max(1, std::min((int)(160 * 1024 / lds), 16 / wk));
        const double rounds = wgs / (256.0 * per_cu);
        const double tail = std::ceil(rounds) / std::max(rounds, 1e-9);
        const double pad = (double)row_blocks * rt / n_tiles;
        const int depth = 8 / rt;
        double score = 0.0;
        score -= (waves < 4096 ? (4096.0 / waves) : 1.0) * 2.0;
        score -= (rounds >= 1.0 ? (tail - 1.0) * 3.0 : 0.0);
        score -= (pad - 1.0) * 4.0;
        score -= (kwmax < depth ? (depth - kwmax) * 0.3 : 0.0);
        score -= (kwmax > 16 ? (kwmax - 16) * 0.02 : 0.0);
        score -= 0.2 * (rows * 2.0) / (rt * 16.0 * 0.5625);
        if (score > best_score) {
          best_score = score;
          best.dot = 1; best.rt = rt; best.wk = wk; best.kw = kwmax; best.win = kwmax;
          best.lds_rows = rows; best.lds_ld = kwmax * kc + 8; best.wave_lds = (int)wl; best.lds_bytes = lds;
        }
      }
    }
    return best;
  }
  for (int rt : {1, 2, 4}) {
    if (force[0] && rt != force[0]) continue;
    for (int wk = 1; wk <= 8; ++wk) {
      if (chunks % wk) continue;
      if (force[0] && wk != force[1]) continue;
      const int kw = chunks / wk;
      for (int win = kw; win >= 1; --win) {
        if (force[0] && win != std::min(force[2], kw)) continue;
        const size_t wl = wave_lds_for(fmt, rows, win * kc);
        const size_t lds = std::max((size_t)wk * wl, (size_t)wk * rt * 64 * 16) + (size_t)wk * 16 * 4 + 64;
        if (lds > kLdsBudget) continue;
        const int nwin = (kw + win - 1) / win;
        const int row_blocks = (n_tiles + rt - 1) / rt;
        const double wgs = (double)row_blocks * groups;
        const double waves = wgs * wk;
        const int per_cu = std::max(1, std::min((int)(160 * 1024 / lds), 16 / wk));
        const double rounds = wgs / (256.0 * per_cu);
        const double tail = std::ceil(rounds) / std::max(rounds, 1e-9);
        const double pad = (double)row_blocks * rt / n_tiles;
        const int depth = 8 / rt;
        double score = 0.0;
        score -= (waves < 4096 ? (4096.0 / waves) : 1.0) * 2.0;          // starved for parallelism
        score -= (rounds >= 1.0 ? (tail - 1.0) * 3.0 : 0.0);
        score -= (pad - 1.0) * 4.0;
        score -= (nwin - 1) * 0.4;                                        // each extra window drains the ring
        score -= (kw < depth ? (depth - kw) * 0.3 : 0.0);                 // prefetch ring not filled
        score -= (kw > 16 ? (kw - 16) * 0.02 : 0.0);                      // long slices: coarse tail
        // activation staging relative to weight bytes streamed per wave: rows·2 per column vs rt·16·0.5625
        score -= 0.6 * (rows * 2.0) / (rt * 16.0 * 0.5625);
        if (score > best_score) {
          best_score = score;
          best.dot = 0; best.rt = rt; best.wk = wk; best.kw = kw; best.win = win;
          best.lds_rows = rows; best.lds_ld = win * kc + 8; best.wave_lds = (int)wl; best.lds_bytes = lds;
        }
        break;   // the widest window that fits is the one to use for this (rt, wk)
      }
    }
  }
  return best;
}

template <int FMT, int RT>
void launch(const Args& a, const Plan& p, dim3 grid, hipStream_t s) {
  if (p.dot) {
    if (p.lds_rows <= 1) hipLaunchKernelGGL((gemv_dot<FMT, RT, 1>), grid, dim3(64 * p.wk), p.lds_bytes, s, a);
    else hipLaunchKernelGGL((gemv_dot<FMT, RT, 2>), grid, dim3(64 * p.wk), p.lds_bytes, s, a);
  } else {
    hipLaunchKernelGGL((gemv_t16<FMT, RT>), grid, dim3(64 * p.wk), p.lds_bytes, s, a);
  }
}

}  // namespace

extern "C" {

size_t mi_pack_bytes(int32_t format, int32_t n, int32_t k) {
  if (n <= 0 || k <= 0) return 0;
  const int kc = chunk_cols(format);
  if (k % kc) return 0;
  return (size_t)((n + 15) / 16) * (k / kc) * unit_bytes(format);
}

size_t mi_gemv_workspace_bytes(const mi_gemv_desc* d) {
  (void)d;
  return 0;
}

int mi_gemv_plan(const mi_gemv_desc* d, int32_t out[7]) {
  if (int rc = check_desc(d)) return rc;
  MI_REQUIRE(out, "mi_gemv_plan: null output");
  const Plan p = make_plan(d);
  MI_REQUIRE(p.kw > 0, "mi_gemv_plan: no launch plan fits (k=%d, m=%d)", d->k, d->m);
  const int n_tiles = (d->n + 15) / 16;
  const int row_blocks = (n_tiles + p.rt - 1) / p.rt;
  out[0] = p.rt; out[1] = p.wk; out[2] = p.kw; out[3] = p.win; out[4] = p.dot ? -1 : (p.kw + p.win - 1) / p.win;
  out[5] = (int32_t)p.lds_bytes; out[6] = row_blocks * (d->groups ? d->max_groups : 1);
  return MI_OK;
}

int mi_gemv(const mi_gemv_desc* d, void* stream) {
  if (int rc = check_desc(d)) return rc;
  const Plan p = make_plan(d);
  MI_REQUIRE(p.kw > 0, "mi_gemv: no launch plan fits (k=%d, m=%d)", d->k, d->m);
  Args a{};
  a.w = static_cast<const uint8_t*>(d->w);
  a.row_scale = d->row_scale;
  a.x = d->x;
  a.y = d->y;
  a.res = d->residual;
  a.norm_w = d->norm_w;
  a.groups = d->groups;
  a.eps = d->eps;
  a.ldx = d->ldx; a.ldy = d->ldy; a.ldr = d->ldr;
  a.n = d->n; a.k = d->k; a.m = d->m;
  a.n_tiles = (d->n + 15) / 16;
  a.chunks = d->k / chunk_cols(d->format);
  a.row_blocks = (a.n_tiles + p.rt - 1) / p.rt;
  a.kw = p.kw; a.win = p.win; a.wave_lds = p.wave_lds;
  a.epilogue = d->epilogue;
  a.top_k = d->top_k;
  a.x_per_slot = d->x_per_slot;
  a.out_f32 = d->out_f32;
  a.lds_rows = p.lds_rows;
  a.lds_ld = p.lds_ld;
  a.expert_stride = (long long)a.n_tiles * a.chunks * unit_bytes(d->format);
  const dim3 grid(a.row_blocks, d->groups ? d->max_groups : 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (d->format * 8 + p.rt) {
    case FMT_NVFP4 * 8 + 1: launch<FMT_NVFP4, 1>(a, p, grid, s); break;
    case FMT_NVFP4 * 8 + 2: launch<FMT_NVFP4, 2>(a, p, grid, s); break;
    case FMT_NVFP4 * 8 + 4: launch<FMT_NVFP4, 4>(a, p, grid, s); break;
    case FMT_INT4 * 8 + 1: launch<FMT_INT4, 1>(a, p, grid, s); break;
    case FMT_INT4 * 8 + 2: launch<FMT_INT4, 2>(a, p, grid, s); break;
    case FMT_INT4 * 8 + 4: launch<FMT_INT4, 4>(a, p, grid, s); break;
    case FMT_BF16 * 8 + 1: launch<FMT_BF16, 1>(a, p, grid, s); break;
    case FMT_BF16 * 8 + 2: launch<FMT_BF16, 2>(a, p, grid, s); break;
    default: launch<FMT_BF16, 4>(a, p, grid, s); break;
  }
  MI_TRY_HIP(hipGetLastError(), "gemv_t16 launch");
  return MI_OK;
}

int mi_dequant(int32_t format, const void* w, const float* row_scale, int32_t n, int32_t k, float* out, void* stream) {
  MI_REQUIRE(w && out, "mi_dequant: null pointer");
  MI_REQUIRE(format == FMT_NVFP4 || format == FMT_INT4 || format == FMT_BF16, "mi_dequant: unknown format");
  const int kc = chunk_cols(format);
  MI_REQUIRE(n > 0 && k > 0 && k % kc == 0, "mi_dequant: bad shape");
  const int chunks = k / kc, tiles = (n + 15) / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  if (format == FMT_NVFP4)
    hipLaunchKernelGGL(dequant_t16<FMT_NVFP4>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  else if (format == FMT_INT4)
    hipLaunchKernelGGL(dequant_t16<FMT_INT4>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  else
    hipLaunchKernelGGL(dequant_t16<FMT_BF16>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  MI_TRY_HIP(hipGetLastError(), "dequant_t16 launch");
  return MI_OK;
}

}  // extern "C"
