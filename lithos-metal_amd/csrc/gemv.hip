// GEMV / skinny GEMM over the T16 weight pack, for M = 1 decode and M ≤ 16 verify, dense or grouped by expert.
//
// Semantics (ops/gemv.py:1-12, nn/linear.py:114-135, kernels/common/gemv_T.metal:232-587): y[t][n] = Σ_k x[t][k]·W[n][k]
// with FP32 accumulation and one BF16 rounding, optional RMSNorm on the input (norm_apply fused on load,
// ops/norm.py:1-6) and a residual / silu·mul epilogue. Grouped mode is the MoE expert GEMV (ops/moe.py `moe_gemv`):
// a group is one expert with the ≤ 16 (token, slot) pairs routed to it, so a step streams exactly the chosen experts.
//
// MI355X design. The pack streams 16-row tiles in 128-column chunks; lane l of a wave owns row l%16 and the 32
// columns 32·(l/16)… of a chunk, one fully coalesced 1 KiB load per chunk (NVFP4 block scales: one 16-byte load per
// 8 chunks). What sets the speed is how many of those loads are in flight per CU and how cheaply the activations
// reach every wave; two kernels:
//  * gemv_row (M <= 2): a workgroup per tile, its waves splitting K into slices of KW = 4/8/16 chunks; each wave
//    issues its activation slice, the slice's scales and all KW weight chunks at once, stages the activations in its
//    own LDS region, and computes on the VALU: NVFP4 → BF16 pairs with v_cvt_scalef32_pk_bf16_fp4 (e2m1 × the power-
//    of-two part of the E4M3 block scale, exact), v_dot2_f32_bf16 against the BF16 activations as they are, the
//    scale's 3-bit mantissa applied once per block of 16; INT4 as BF16 128 + c corrected by 128·Σx per segment. The
//    K slices meet in LDS (fixed order). Many short waves keep ~all weight bytes of the CU's share in flight.
//    gemv_rowp is the same wave layout looping over several tiles per workgroup, for a fused input norm over many
//    tiles: the norm's statistic (a workgroup barrier on the critical path of every workgroup) is then paid once
//    per workgroup instead of once per tile.
//  * gemv_tk (M ≤ 16): MFMA v_mfma_f32_16x16x32_{f16,bf16} with the activations as the A operand (token rows,
//    power-of-two prescaled into F16 range: exact above 2^-14 of the row max) and the decoded weights as B (NVFP4 →
//    exact F16 by v_cvt_scalef32_pk_f16_fp4 and a packed multiply by the mantissa factor). A workgroup stages one K
//    split of the activations once and streams many tiles against it, so the activations are re-read per workgroup,
//    not per tile; long K is split across workgroups with FP32 partials added in order by gemv_tk_reduce.
// Cross-workgroup reduction: gemv_row with split K folds its splits in the kernel (the last split of a tile to
// arrive adds them in split order) through device-scope atomic read-modify-writes only, with no release / acquire
// fence — on gfx950 such a fence writes back / invalidates the whole L2 per workgroup and costs more than the GEMV.
// gemv_tk and gemv_rowm leave their split partials to the ordered gemv_tk_reduce launch.
#include "mi_common.h"
#include "route.h"
#include "t16.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <type_traits>
#include <mutex>
#include <tuple>
#include <vector>

namespace {

struct Args {
  const uint8_t* w;
  const float* row_scale;
  const uint16_t* x;
  uint16_t* y;
  const uint16_t* res;
  const float* norm_w;
  const int32_t* groups;
  long long expert_stride;  // bytes between experts' packs
  long long tile_stride;    // bytes per tile
  float eps;
  int ldx, ldy, ldr;
  int n, k, m;
  int n_tiles, chunks;
  int epilogue, top_k, x_per_slot, out_f32;
  int lds_rows;             // gemv_tk: staged token rows
  int tb;                   // gemv_tk: 16-row tiles per workgroup
  int ks, kc;               // gemv_tk: K splits, chunks per split
  float* part;              // gemv_tk with ks > 1: FP32 partials [ks][m][n_tiles·16]
  uint32_t* fold_cnt;       // gemv_row with ks > 1: per-tile arrival counters (zero between calls): the last split
                            // of a tile folds the partials in the kernel; null: gemv_tk_reduce does it
  const float* gnorm_w;     // gated head RMSNorm on the input (Gated DeltaNet output norm), or null
  const uint16_t* gnorm_z;
  int ld_gnorm_z;
  float gnorm_eps;
  int row_ld;               // gemv_row: LDS row stride of a wave's staged slice (elements)
  int row_wave_lds;         // gemv_row: LDS bytes per wave
  int shared_expert, shared_epilogue;   // grouped: the shared expert's group takes its own epilogue (0 = none)
  // grouped, one token: the launch routes for itself (group g = slot g of the token's top-k, the shared expert
  // last) from the router's logits row, and its first workgroup writes the route (ids, weights, groups) for the
  // launches after it
  const uint16_t* route_logits;
  int route_e, route_k, route_renorm, route_gate_col, route_n;   // route_n: group records to write
  int32_t* route_ids;
  float* route_weights;
  int32_t* route_groups;
  int passes;               // gemv_row, dense M > 2: tokens taken MT per workgroup along grid z (0 / 1: none)
  // gemv_row, M <= 2: the Gated DeltaNet short conv over output rows conv_row0 .. conv_row0 + conv_ch (null conv_w:
  // off); the state in conv_in (two slots chosen by *conv_step when given) → conv_out_state, outputs in conv_out
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out_state;
  uint16_t* conv_out;
  int conv_row0, conv_ch, ld_conv;
  const uint32_t* conv_step;
  const uint32_t* conv_done;
  // dense, BF16 output: the next RMSNorm of y (x_next = bf16(y·rsqrt(mean y² + eps)·w)) computed by the split-K
  // reduction (gemv_reduce_norm); null: off
  const float* nn_w;
  uint16_t* nn_x;
  int ld_nn_x;
  float nn_eps;
};

// The conv's per-row inputs, loaded at the start of the launch (independent of the GEMV): the 4 taps, the W-1 = 3
// state inputs of both slots (the slot is chosen by value, so every load is unconditional), the step and stop words
struct ConvIn {
  uint2 w;
  uint16_t s[2][3];
  uint32_t step, done;
};

__device__ __forceinline__ void conv_load(const Args& a, int ch, ConvIn& c) {
  c.w = *reinterpret_cast<const uint2*>(a.conv_w + (long long)ch * 4);
  const uint16_t* s1 = a.conv_step ? a.conv_in + (long long)a.conv_ch * 3 : a.conv_in;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    c.s[0][j] = a.conv_in[(long long)ch * 3 + j];
    c.s[1][j] = s1[(long long)ch * 3 + j];
  }
  c.step = a.conv_step ? *a.conv_step : 0u;
  c.done = a.conv_done ? *a.conv_done : 0u;
}

// Channel ch's conv over [3 state inputs | the cnt new outputs x (BF16-valued)]: out_t = bf16(silu(bf16(Σ_j w_j·
// x_{t+j}))), summed in tap order as the oracle (and gdn_step's own conv) does; the new state is the last 3 inputs.
// Stopped (done): the state passes to the output slot unchanged and nothing else is written.
template <int MT>
__device__ __forceinline__ void conv_emit(const Args& a, int ch, const ConvIn& c, const float (&x)[MT], int cnt) {
  const uint32_t rd = a.conv_step ? (c.step & 1u) : 0u;
  uint16_t* sout = a.conv_step ? const_cast<uint16_t*>(a.conv_in) + (long long)(rd ^ 1u) * a.conv_ch * 3
                               : a.conv_out_state;
  float xs[3 + MT];
#pragma unroll
  for (int j = 0; j < 3; ++j) xs[j] = bf16_bits_to_f32(rd ? c.s[1][j] : c.s[0][j]);
  const int T = c.done ? 0 : cnt;
#pragma unroll
  for (int t = 0; t < MT; ++t) xs[3 + t] = t < T ? x[t] : 0.0f;
  const float w[4] = {bf16_bits_to_f32(c.w.x & 0xFFFFu), bf16_bits_to_f32(c.w.x >> 16),
                      bf16_bits_to_f32(c.w.y & 0xFFFFu), bf16_bits_to_f32(c.w.y >> 16)};
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    if (t >= T) break;
    float y = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) y = __fadd_rn(y, __fmul_rn(w[j], xs[j + t]));
    a.conv_out[(long long)t * a.ld_conv + ch] = f32_to_bf16_bits(silu_f(round_bf16(y)));
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    float v = xs[j];
#pragma unroll
    for (int t = 1; t <= MT; ++t) v = (t == T) ? xs[t + j] : v;
    sout[(long long)ch * 3 + j] = f32_to_bf16_bits(v);
  }
}

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
  s.m0 = (f16_t)nv_mant(u0);   // ±1.mmm, exact in F16
  s.m1 = (f16_t)nv_mant(u1);
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

// FP8 E4M3: codes 2j, 2j+1 of a dword (hi: 2, 3) → exact BF16 / F16 pairs (scale 1: the tensor scale is the row's)
__device__ __forceinline__ bf16x2 cvt_fp8x2_bf16(uint32_t dw, bool hi) {
  return hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(dw, 1.0f, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(dw, 1.0f, false);
}
__device__ __forceinline__ f16x8 fp8_decode8(uint32_t d0, uint32_t d1) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, false), b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, true);
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, false), e = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, true);
  return f16x8{a.x, a.y, b.x, b.y, c.x, c.y, e.x, e.y};
}

__device__ __forceinline__ int int4_perm8(int i) { return (i & 1) ? 4 + (i >> 1) : (i >> 1); }


__device__ __forceinline__ void store_out(const Args& a, long long idx, float v) {
  if (a.out_f32) reinterpret_cast<float*>(a.y)[idx] = v;
  else a.y[idx] = f32_to_bf16_bits(v);
}


// one output value: row tile·16 + m_row of token t, already scaled by its row scale; `up` is the value of the row
// 8 below it (the up half of a silu·mul tile), fetched by the caller with a shuffle every lane executes
// the epilogue of a workgroup's matrix: the descriptor's, or the shared expert's for its group
__device__ __forceinline__ int epilogue_of(const Args& a, int expert) {
  return a.shared_expert > 0 && expert == a.shared_expert ? a.shared_epilogue : a.epilogue;
}

__device__ __forceinline__ void emit_row(const Args& a, int epi, int yr, int cnt, int tile, bool tile_ok, int m_row,
                                         int t, float v, float up);
__device__ __forceinline__ void emit(const Args& a, int epi, const int32_t* pairs, int cnt, int tile, bool tile_ok,
                                     int m_row, int t, float v, float up) {
  if (!tile_ok || t >= cnt) return;
  emit_row(a, epi, pairs ? pairs[t] : t, cnt, tile, tile_ok, m_row, t, v, up);
}

// the same with token t's output row yr given
__device__ __forceinline__ void emit_row(const Args& a, int epi, int yr, int cnt, int tile, bool tile_ok, int m_row,
                                         int t, float v, float up) {
  if (!tile_ok || t >= cnt) return;
  if (epi == MI_EPI_SILU_MUL || epi == MI_EPI_SILU_MUL_ROUNDED) {
    const int col = tile * 8 + m_row;
    if (m_row >= 8 || col >= a.n / 2) return;
    float o;
    if (epi == MI_EPI_SILU_MUL_ROUNDED) {
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
    if (epi == MI_EPI_RESIDUAL) o += bf16_bits_to_f32(a.res[(long long)yr * a.ldr + row]);   // dense: yr = token
    store_out(a, (long long)yr * a.ldy + row, o);
  }
}


// ---- one chunk of one tile in registers ---------------------------------------------------------------------
// 16 bytes of streamed weights: read once per launch, so loaded non-temporally (they need not stay in the caches)
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint8_t* p) {
#ifdef MI_WEIGHTS_TEMPORAL
  return *reinterpret_cast<const uint4*>(p);
#else
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return uint4{v.x, v.y, v.z, v.w};
#endif
}

template <int FMT>
struct Units {
  uint4 q;                   // lane l: 16 bytes of codes (NVFP4 / INT4) or 8 BF16 values
  uint32_t s;                // NVFP4 (gemv_tk): the lane's two E4M3 block-scale bytes
  uint2 sb;                  // INT4: (scale, bias) pairs of the chunk's two groups
};

// chunk c of the tile at `tb`; NVFP4 scales for gemv_tk from the group's scale block (gemv_row loads whole pieces)
template <int FMT, bool SCALE>
__device__ __forceinline__ void load_chunk(Units<FMT>& u, const uint8_t* tb, int c, int chunks, int lane) {
  if constexpr (FMT == FMT_NVFP4) {
    u.q = ld_stream(tb + nv_code_off(c) + 16 * lane);
    if constexpr (SCALE) {
      const int gi = c >> 3;
      u.s = *reinterpret_cast<const uint16_t*>(tb + nv_scale_off(gi, chunks) + nv_piece(nv_group_chunks(gi, chunks)) * lane +
                                               2 * (c & 7));
    }
  } else {
    const uint8_t* p = tb + (long long)c * unit_bytes(FMT);
    u.q = ld_stream(p + 16 * lane);
    if constexpr (FMT == FMT_INT4) u.sb = *reinterpret_cast<const uint2*>(p + 1024 + 8 * (lane & 15));
  }
}

// ---- gemv_row: M <= 2 ------------------------------------------------------------------------------------------
// Workgroup = one 16-row tile (blockIdx.x) of one group (blockIdx.y, MoE); wave w = K slice [w·KW, w·KW + KW).
// LDS: per wave xs[MT][row_ld] (INT4: then seg[MT][KW][8]) | stat[S][2] | red[S][MT][16].
// CONV: the launch carries the GDN conv epilogue (a separate instantiation: its registers and code stay out of the
// plain GEMV, whose occupancy they would otherwise cut).
template <int FMT, int MT, int KW, bool CONV>
__global__ __launch_bounds__(KW == 16 ? 640 : 1024) void gemv_row(Args a) {
  constexpr int KC = chunk_cols(FMT);
  constexpr int NPL = MT * KW * KC / 8 / 64 > 0 ? MT * KW * KC / 8 / 64 : 1;   // activation vectors per lane
  constexpr int NG = FMT == FMT_NVFP4 ? (KW + 7) / 8 : 0;                         // scale pieces per wave
  static_assert(KW == 4 || KW % 8 == 0, "NVFP4 slices: half a scale group or whole groups");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (scalar) in the compiler's view
  const int S = blockDim.x >> 6;
  const int tile = blockIdx.x;
  int expert = 0, cnt = a.m;
  const int32_t* pairs = nullptr;
  __shared__ int route_sel[ROUTE_MAX_K + 2];    // routing for itself: the slots' experts, then this group's pair
  if (a.route_logits) {                         // workgroup-uniform: one token, group g = slot g
    if (wave == 0) {
      int ce[ROUTE_MAX_K];
      float cw[ROUTE_MAX_K];
      route_topk(a.route_logits, a.route_e, a.route_k, a.route_renorm, lane, ce, cw);
      const int k = a.route_k, ks = k + (a.shared_expert > 0 ? 1 : 0);
      if (lane == 0) {
        for (int r = 0; r < k; ++r) route_sel[r] = ce[r];
        if (ks > k) route_sel[k] = a.shared_expert;
        route_sel[ROUTE_MAX_K + 1] = blockIdx.y;
        if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) {   // the route for the launches after this one
          for (int r = 0; r < k; ++r) {
            a.route_ids[r] = ce[r];
            a.route_weights[r] = cw[r];
          }
          if (ks > k) {
            a.route_ids[k] = a.shared_expert;
            a.route_weights[k] = route_shared_weight(bf16_bits_to_f32(a.route_logits[a.route_gate_col]));
          }
          for (int r = 0; r < a.route_n; ++r) {                          // record r = slot r (pair r)
            int32_t* rec = a.route_groups + r * GROUP_REC;
            const int e = r < ks ? (r < k ? ce[r] : a.shared_expert) : -1;
            rec[0] = e;
            rec[1] = e >= 0 ? 1 : 0;
            rec[2] = r;
          }
        }
      }
    }
    __syncthreads();
    expert = route_sel[blockIdx.y];
    cnt = 1;
    pairs = &route_sel[ROUTE_MAX_K + 1];
    if (expert < 0) return;                   // a slot without an expert (NaN logits): the workgroup leaves
  } else if (a.groups) {
    const int32_t* g = a.groups + blockIdx.y * GROUP_REC;
    expert = g[0];
    cnt = g[1];
    pairs = g + 2;
    if (cnt <= 0 || expert < 0) return;       // the whole workgroup leaves together
  }
  // more than MT tokens (a grouped launch's pairs, or a.passes > 1 dense tokens) are taken MT per workgroup, pass
  // blockIdx.z (one K split); a pass past the tokens leaves at once
  const bool zpass = (a.groups && !a.route_logits) || a.passes > 1;
  const int pass = zpass ? (int)blockIdx.z : 0;
  if (pass * MT >= cnt) return;                 // workgroup-uniform
  if (pairs) pairs += pass * MT;
  cnt = min(MT, cnt - pass * MT);
  const int t0 = pairs ? 0 : pass * MT;         // dense: the pass's first token
  const long long xr0 = pairs ? (a.x_per_slot ? pairs[0] : pairs[0] / a.top_k) : t0;
  const long long xr1 = MT > 1 ? (pairs ? (a.x_per_slot ? pairs[cnt - 1] : pairs[cnt - 1] / a.top_k) : t0 + cnt - 1) : 0;
  const int split = zpass ? 0 : (int)blockIdx.z;   // K split (a.ks of a.kc chunks each; FP32 partials when > 1)
  const int c0_raw = split * a.kc + wave * KW;
  const int kw = min(KW, min(a.chunks, (split + 1) * a.kc) - c0_raw);   // <= 0: a wave past a short last split
  const int c0 = kw > 0 ? c0_raw : 0;           // such a wave reads chunk 0 (in bounds) and adds nothing
  const int kwl = max(kw, 1);
  const int cols = kwl * KC;
  const uint8_t* tbase = a.w + (long long)expert * a.expert_stride + (long long)tile * a.tile_stride;
  // the conv's inputs for wave 0's rows (a tile lies wholly inside or outside the conv channels): issued first,
  // used in the epilogue
  const bool conv_tile = CONV && tile * 16 >= a.conv_row0 && tile * 16 < a.conv_row0 + a.conv_ch;
  ConvIn cvin{};
  if constexpr (CONV) {
    if (conv_tile && wave == 0) conv_load(a, tile * 16 + (lane & 15) - a.conv_row0, cvin);
  }

  // ---- loads: activations, norm weights, scale pieces, then every weight chunk of the slice --------------------
  const int per_row = cols / 8;
  uint4 xv[NPL], zv[NPL];
  float4 nv[NPL][2];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int idx = min(lane + 64 * i, MT * per_row - 1);
    const int j = MT > 1 && idx >= per_row ? 1 : 0;
    const int e = (idx - j * per_row) * 8;
    xv[i] = *reinterpret_cast<const uint4*>(a.x + (j ? xr1 : xr0) * a.ldx + c0 * KC + e);
    if (a.norm_w) {
      nv[i][0] = *reinterpret_cast<const float4*>(a.norm_w + c0 * KC + e);
      nv[i][1] = *reinterpret_cast<const float4*>(a.norm_w + c0 * KC + e + 4);
    } else if (a.gnorm_w) {
      zv[i] = *reinterpret_cast<const uint4*>(a.gnorm_z + (j ? xr1 : xr0) * a.ld_gnorm_z + c0 * KC + e);
      nv[i][0] = *reinterpret_cast<const float4*>(a.gnorm_w + ((c0 * KC + e) & 127));
      nv[i][1] = *reinterpret_cast<const float4*>(a.gnorm_w + ((c0 * KC + e) & 127) + 4);
    }
  }
  uint4 sv[NG > 0 ? NG : 1];
  if constexpr (FMT == FMT_NVFP4) {
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const int gi = min((c0 >> 3) + q, (a.chunks - 1) >> 3);
      const int gsz = nv_group_chunks(gi, a.chunks);
      const uint8_t* p = tbase + nv_scale_off(gi, a.chunks);
      if (nv_piece(gsz) == 16) {
        sv[q] = *reinterpret_cast<const uint4*>(p + 16 * lane);
      } else {
        const uint2 t = *reinterpret_cast<const uint2*>(p + 8 * lane);
        sv[q] = uint4{t.x, t.y, 0u, 0u};
      }
    }
  }
  Units<FMT> u[KW];
#pragma unroll
  for (int cc = 0; cc < KW; ++cc) load_chunk<FMT, false>(u[cc], tbase, c0 + min(cc, kwl - 1), a.chunks, lane);

  // ---- stage the slice (normalized when the norm is fused: Σh² over the row from every wave's slice) ----------
  uint8_t* wl = smem + (size_t)wave * a.row_wave_lds;
  uint16_t* xs = reinterpret_cast<uint16_t*>(wl);
  const int ld = a.row_ld;
  float* seg = reinterpret_cast<float*>(wl + (size_t)MT * ld * 2);
  float* stat = reinterpret_cast<float*>(smem + (size_t)S * a.row_wave_lds);   // [S][2]
  float* red = stat + 2 * S;                                                  // [S][MT][16]
  if (a.norm_w) {
    float sq[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int idx = lane + 64 * i;
      if (idx < MT * per_row) {
        const uint32_t vv[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        float t = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bf16_bits_to_f32(vv[q] & 0xFFFFu), hi = bf16_bits_to_f32(vv[q] >> 16);
          t = fmaf(lo, lo, fmaf(hi, hi, t));
        }
        sq[MT > 1 && idx >= per_row ? 1 : 0] += t;
      }
    }
    sq[0] = wave_sum(sq[0]);
    if (MT > 1) sq[1] = wave_sum(sq[1]);
    if (lane == 0) { stat[2 * wave] = sq[0]; stat[2 * wave + 1] = sq[1]; }
    __syncthreads();
    float rstd[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float t = 0.0f;
      for (int w = 0; w < S; ++w) t += stat[2 * w + j];
      rstd[j] = 1.0f / sqrtf(t / (float)a.k + a.eps);
    }
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int idx = lane + 64 * i;
      const float rr = rstd[MT > 1 && idx >= per_row ? 1 : 0];
      const float wv[8] = {nv[i][0].x, nv[i][0].y, nv[i][0].z, nv[i][0].w, nv[i][1].x, nv[i][1].y, nv[i][1].z, nv[i][1].w};
      uint32_t* vv = reinterpret_cast<uint32_t*>(&xv[i]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = round_bf16((bf16_bits_to_f32(vv[q] & 0xFFFFu) * rr) * wv[2 * q]);
        const float hi = round_bf16((bf16_bits_to_f32(vv[q] >> 16) * rr) * wv[2 * q + 1]);
        vv[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
      }
    }
  } else if (a.gnorm_w) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) gated_head_norm8(reinterpret_cast<uint32_t(&)[4]>(xv[i]), zv[i], nv[i][0], nv[i][1], a.gnorm_eps);
  }
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int idx = lane + 64 * i;
    if (idx < MT * per_row) {
      const int j = MT > 1 && idx >= per_row ? 1 : 0;
      uint4 v = xv[i];
      if constexpr (FMT == FMT_INT4) {        // (x0,x1)(x2,x3)(x4,x5)(x6,x7) → (x0,x4)(x1,x5)(x2,x6)(x3,x7)
        const uint32_t a0 = v.x, a1 = v.y, a2 = v.z, a3 = v.w;
        v.x = __builtin_amdgcn_perm(a2, a0, 0x05040100u);
        v.y = __builtin_amdgcn_perm(a2, a0, 0x07060302u);
        v.z = __builtin_amdgcn_perm(a3, a1, 0x05040100u);
        v.w = __builtin_amdgcn_perm(a3, a1, 0x07060302u);
      }
      *reinterpret_cast<uint4*>(xs + (size_t)j * ld + (idx - j * per_row) * 8) = v;
    }
  }
  wave_lds_sync();
  if constexpr (FMT == FMT_INT4) {
    // Σx over each (chunk, g, group) segment of 16 columns: steps {0,1} (group A) / {2,3} (group B) of k-group g
    for (int idx = lane; idx < MT * KW * 8; idx += 64) {
      const int j = idx / (KW * 8), rem = idx - j * KW * 8;
      const int cc = rem >> 3, g = (rem >> 1) & 3, gp = rem & 1;
      float sx = 0.0f;
      if (cc < kw) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const uint4 v = *reinterpret_cast<const uint4*>(xs + (size_t)j * ld + cc * 128 + 32 * (2 * gp + st) + 8 * g);
          const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) sx += bf16_bits_to_f32(vv[q] & 0xFFFFu) + bf16_bits_to_f32(vv[q] >> 16);
        }
      }
      seg[idx] = sx;
    }
    wave_lds_sync();
  }

  // ---- the slice's dot products --------------------------------------------------------------------------------
  const int g = lane >> 4, m_row = lane & 15;
  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
  auto slice_chunk = [&](int cc) {
    const uint32_t dw[4] = {u[cc].q.x, u[cc].q.y, u[cc].q.z, u[cc].q.w};
    if constexpr (FMT == FMT_NVFP4) {
      uint4 xq[MT][4];
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * g + 8 * s);
      // chunk in its group: KW >= 8 slices start on a group, KW = 4 slices on one of its halves (c0 % 4 == 0)
      const uint4 pv = sv[KW >= 8 ? cc >> 3 : 0];
      const uint32_t word = KW >= 8 ? (cc & 6) == 0 ? pv.x : (cc & 6) == 2 ? pv.y : (cc & 6) == 4 ? pv.z : pv.w
                                    : (c0 & 4) ? (cc < 2 ? pv.z : pv.w) : (cc < 2 ? pv.x : pv.y);
      const f32x2 f = (cc & 1) ? __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true)
                               : __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
      const uint32_t u0 = __float_as_uint(f.x), u1 = __float_as_uint(f.y);
      const float e[2] = {__uint_as_float(u0 & 0x7F800000u), __uint_as_float(u1 & 0x7F800000u)};
      const float mant[2] = {nv_mant(u0),
                             nv_mant(u1)};
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float part[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) part[t] = 0.0f;
#pragma unroll
        for (int s = 2 * b; s < 2 * b + 2; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x2 w2 = cvt_fp4x2_bf16(dw[s], e[b], j);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
              const uint32_t xw = j == 0 ? xq[t][s].x : j == 1 ? xq[t][s].y : j == 2 ? xq[t][s].z : xq[t][s].w;
              part[t] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf16x2, xw), part[t], false);
            }
          }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = fmaf(part[t], mant[b], acc[t]);
      }
    } else if constexpr (FMT == FMT_INT4) {
      uint4 xq[MT][4];
      float sa[MT], sb[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int s = 0; s < 4; ++s) xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * s + 8 * g);
        sa[t] = seg[(t * KW + cc) * 8 + g * 2];
        sb[t] = seg[(t * KW + cc) * 8 + g * 2 + 1];
      }
      float d[2][MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) d[0][t] = d[1][t] = 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
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
      const float sca = bf16_bits_to_f32(u[cc].sb.x & 0xFFFFu), bia = bf16_bits_to_f32(u[cc].sb.x >> 16);
      const float scb = bf16_bits_to_f32(u[cc].sb.y & 0xFFFFu), bib = bf16_bits_to_f32(u[cc].sb.y >> 16);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        acc[t] = fmaf(sca, fmaf(-128.0f, sa[t], d[0][t]), fmaf(bia, sa[t], acc[t]));
        acc[t] = fmaf(scb, fmaf(-128.0f, sb[t], d[1][t]), fmaf(bib, sb[t], acc[t]));
      }
    } else if constexpr (FMT == FMT_FP8) {
      uint4 xq[MT][2];                      // the lane's 16 columns 64·cc + 16·g + [0, 16)
    #pragma unroll
      for (int t = 0; t < MT; ++t)
    #pragma unroll
        for (int h = 0; h < 2; ++h) xq[t][h] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 64 + 16 * g + 8 * h);
    #pragma unroll
      for (int q = 0; q < 4; ++q)
    #pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
          const bf16x2 w2 = cvt_fp8x2_bf16(dw[q], hi);   // columns 4q + 2hi, +1 of the lane's 16
    #pragma unroll
          for (int t = 0; t < MT; ++t) {
            const uint4 xv4 = xq[t][q >> 1];
            const int e = 2 * (q & 1) + hi;
            const uint32_t xw = e == 0 ? xv4.x : e == 1 ? xv4.y : e == 2 ? xv4.z : xv4.w;
            acc[t] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf16x2, xw), acc[t], false);
          }
        }
    } else {
      uint4 xq[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) xq[t] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 32 + 8 * g);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint32_t xw = j == 0 ? xq[t].x : j == 1 ? xq[t].y : j == 2 ? xq[t].z : xq[t].w;
          acc[t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, dw[j]), __builtin_bit_cast(bf16x2, xw),
                                                   acc[t], false);
        }
    }
  };
#pragma unroll
  for (int cc = 0; cc < KW; ++cc)
    if (cc < kw) slice_chunk(cc);

  // ---- the four k-groups of each row, then the K slices in wave order, then the epilogue ------------------------
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float v = quad16_sum(acc[t]);
    if (g == 0) red[(wave * MT + t) * 16 + m_row] = v;
  }
  __syncthreads();
  if (wave != 0) return;
  const int row = tile * 16 + m_row;
  float vt[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) vt[t] = slice_sum(red + t * 16, MT * 16, S, lane);
  if (a.ks > 1) {
    const long long pstride = (long long)a.n_tiles * 16;
    if (!a.fold_cnt) {                          // this split's partial; gemv_tk_reduce adds the splits in order
#pragma unroll
      for (int t = 0; t < MT; ++t)
        if (g == 0 && t < cnt) a.part[((long long)split * a.m + t) * pstride + row] = vt[t];
      return;
    }
    // The splits of a tile meet without a memory fence (an agent-scope release writes back the whole L2 — about
    // 0.15 us per workgroup, serialized): partials and counter are device-scope atomic read-modify-writes, performed
    // at the device's coherence point in the order each lane issues them; every exchange has returned before the
    // counter moves, and the last split reads the partials back with read-modify-writes issued after it saw the
    // count. It adds the splits in split order (the result of gemv_tk_reduce, bit for bit) and re-arms the counter.
    auto* pu = reinterpret_cast<uint32_t*>(a.part);
    uint32_t seen = 0;
#pragma unroll
    for (int t = 0; t < MT; ++t)
      if (g == 0 && t < cnt)
        seen |= __hip_atomic_exchange(pu + ((long long)split * a.m + t) * pstride + row, __float_as_uint(vt[t]),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(seen) : "memory");     // the exchanges have returned
    uint32_t prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(a.fold_cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != (uint32_t)(a.ks - 1)) return;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float v = 0.0f;
      if (g == 0 && t < cnt)
        for (int sp = 0; sp < a.ks; ++sp)
          v += __uint_as_float(__hip_atomic_fetch_or(pu + ((long long)sp * a.m + t) * pstride + row, 0u,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      vt[t] = v;
    }
    if (lane == 0) __hip_atomic_store(a.fold_cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const float rs = a.row_scale != nullptr ? a.row_scale[(long long)expert * a.n_tiles * 16 + row] : 1.0f;
  float xb[MT];                                 // the BF16 outputs (the conv's new inputs)
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    float v = vt[t];
    v *= rs;
    xb[t] = round_bf16(v);
    const float up = __shfl_down(v, 8, 16);
    if (g == 0 && t < cnt) emit_row(a, epilogue_of(a, expert), pairs ? pairs[t] : t0 + t, cnt, tile, true, m_row, t, v, up);
  }
  if constexpr (CONV) {
    if (conv_tile && g == 0) conv_emit<MT>(a, row - a.conv_row0, cvin, xb, cnt);
  }
}

// ---- gemv_rowp: M = 1, a workgroup over several tiles ------------------------------------------------------------------------------------------
// Workgroup = S waves over tiles blockIdx.x, blockIdx.x + G, … (G = gridDim.x, at most a.rt tiles; G is sized so
// every workgroup is resident at once) of one group (blockIdx.y, MoE) and one K split (blockIdx.z); wave w owns the
// K slice [w·KW, w·KW + KW) of every one of those tiles. The activations (normalized when the norm is fused) are
// staged once per workgroup; each wave issues tile j + 1 as soon as tile j is consumed. A tile's K slices meet in
// LDS after the last tile, in the order of gemv_row.
// LDS: per wave xs[MT][row_ld] (INT4: then seg[MT][KW][8]) | stat[S][2] | red[rt][S][MT][16].
template <int FMT, int MT, int KW>
__global__ __launch_bounds__(KW == 16 ? 640 : 1024) __attribute__((amdgpu_waves_per_eu(KW == 4 && MT == 1 ? 8 : 1)))
void gemv_rowp(Args a) {
  constexpr int KC = chunk_cols(FMT);
  constexpr int NPL = MT * KW * KC / 8 / 64 > 0 ? MT * KW * KC / 8 / 64 : 1;   // activation vectors per lane
  constexpr int NG = FMT == FMT_NVFP4 ? (KW + 7) / 8 : 1;                         // scale pieces per wave and tile
  static_assert(KW == 4 || KW % 8 == 0, "NVFP4 slices: half a scale group or whole groups");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (scalar) in the compiler's view
  const int S = blockDim.x >> 6;
  const int G = gridDim.x;
  const int ntl = (a.n_tiles - 1 - (int)blockIdx.x) / G + 1;   // this workgroup's tiles (gridDim.x <= n_tiles)
  int expert = 0, cnt = a.m;
  const int32_t* pairs = nullptr;
  if (a.groups) {
    const int32_t* g = a.groups + blockIdx.y * GROUP_REC;
    expert = g[0];
    cnt = g[1];
    pairs = g + 2;
    if (cnt <= 0 || expert < 0) return;       // the whole workgroup leaves together
  }
  if (cnt > MT) cnt = MT;
  const long long xr0 = pairs ? (a.x_per_slot ? pairs[0] : pairs[0] / a.top_k) : 0;
  const long long xr1 = MT > 1 ? (pairs ? (a.x_per_slot ? pairs[cnt - 1] : pairs[cnt - 1] / a.top_k) : cnt - 1) : 0;
  const int split = blockIdx.z;                  // K split (a.ks of a.kc chunks each; FP32 partials when > 1)
  const int c0_raw = split * a.kc + wave * KW;
  const int kw = min(KW, min(a.chunks, (split + 1) * a.kc) - c0_raw);   // <= 0: a wave past a short last split
  const int c0 = kw > 0 ? c0_raw : 0;           // such a wave reads chunk 0 (in bounds) and adds nothing
  const int kwl = max(kw, 1);
  const int cols = kwl * KC;
  const uint8_t* wmat = a.w + (long long)expert * a.expert_stride;
  auto tile_of = [&](int j) { return (int)blockIdx.x + j * G; };

  // ---- loads: activations, norm weights, then the first two tiles' scale pieces and weight chunks -------------
  const int per_row = cols / 8;
  uint4 xv[NPL], zv[NPL];
  float4 nv[NPL][2];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int idx = min(lane + 64 * i, MT * per_row - 1);
    const int j = MT > 1 && idx >= per_row ? 1 : 0;
    const int e = (idx - j * per_row) * 8;
    xv[i] = *reinterpret_cast<const uint4*>(a.x + (j ? xr1 : xr0) * a.ldx + c0 * KC + e);
    if (a.norm_w) {
      nv[i][0] = *reinterpret_cast<const float4*>(a.norm_w + c0 * KC + e);
      nv[i][1] = *reinterpret_cast<const float4*>(a.norm_w + c0 * KC + e + 4);
    } else if (a.gnorm_w) {
      zv[i] = *reinterpret_cast<const uint4*>(a.gnorm_z + (j ? xr1 : xr0) * a.ld_gnorm_z + c0 * KC + e);
      nv[i][0] = *reinterpret_cast<const float4*>(a.gnorm_w + ((c0 * KC + e) & 127));
      nv[i][1] = *reinterpret_cast<const float4*>(a.gnorm_w + ((c0 * KC + e) & 127) + 4);
    }
  }
  // chunk cc of the slice at a compile-time offset from chunk c0 (NVFP4: KW = 4 slices lie in one group of 8,
  // longer ones start on a group); chunks past a short slice are not loaded (their arithmetic is skipped)
  const long long c0_off = FMT == FMT_NVFP4 ? nv_code_off(c0) : (long long)c0 * unit_bytes(FMT);
  auto issue_scales = [&](uint4 (&sv)[NG], int j) {
    const uint8_t* tbase = wmat + (long long)tile_of(j) * a.tile_stride;
    if constexpr (FMT == FMT_NVFP4) {
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        const int gi = min((c0 >> 3) + q, (a.chunks - 1) >> 3);
        const int gsz = nv_group_chunks(gi, a.chunks);
        const uint8_t* p = tbase + nv_scale_off(gi, a.chunks);
        // a group of 8 chunks holds 16 scale bytes a lane, a shorter one 8 (then t1 repeats t0: such a group is
        // one slice, starting on the group, whose chunks use sv.x / sv.y only); both loads unconditional, so no
        // value waits for them at a branch
        const bool wide = nv_piece(gsz) == 16;
        const uint2 t0 = *reinterpret_cast<const uint2*>(p + (wide ? 16 : 8) * lane);
        const uint2 t1 = *reinterpret_cast<const uint2*>(p + (wide ? 16 * lane + 8 : 8 * lane));
        sv[q] = uint4{t0.x, t0.y, t1.x, t1.y};
      }
    }
  };
  // chunk cc of tile j into u[cc] (cc a compile-time index; a chunk past a short slice re-reads the slice's last
  // one, never used: every load unconditional)
  auto issue_chunk = [&](Units<FMT> (&u)[KW], int cc, int j) {
    const int sc = min(cc, kwl - 1);
    const uint8_t* cb = wmat + (long long)tile_of(j) * a.tile_stride + c0_off;
    if constexpr (FMT == FMT_NVFP4) {
      const int off = KW <= 4 ? sc * 1024 : (sc >> 3) * 9216 + (sc & 7) * 1024;
      u[cc].q = ld_stream(cb + off + 16 * lane);
    } else {
      const uint8_t* p = cb + sc * unit_bytes(FMT);
      u[cc].q = ld_stream(p + 16 * lane);
      if constexpr (FMT == FMT_INT4) u[cc].sb = *reinterpret_cast<const uint2*>(p + 1024 + 8 * (lane & 15));
    }
  };
  Units<FMT> u0[KW];
  uint4 s0[NG], s1[NG];
  issue_scales(s0, 0);
#pragma unroll
  for (int cc = 0; cc < KW; ++cc) issue_chunk(u0, cc, 0);

  // ---- stage the slice (normalized when the norm is fused: Σh² over the row from every wave's slice) ----------
  uint8_t* wl = smem + (size_t)wave * a.row_wave_lds;
  uint16_t* xs = reinterpret_cast<uint16_t*>(wl);
  const int ld = a.row_ld;
  float* seg = reinterpret_cast<float*>(wl + (size_t)MT * ld * 2);
  float* stat = reinterpret_cast<float*>(smem + (size_t)S * a.row_wave_lds);   // [S][2]
  float* red = stat + 2 * S;                                                  // [rt][S][MT][16]
  if (a.norm_w) {
    float sq[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int idx = lane + 64 * i;
      if (idx < MT * per_row) {
        const uint32_t vv[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        float t = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bf16_bits_to_f32(vv[q] & 0xFFFFu), hi = bf16_bits_to_f32(vv[q] >> 16);
          t = fmaf(lo, lo, fmaf(hi, hi, t));
        }
        sq[MT > 1 && idx >= per_row ? 1 : 0] += t;
      }
    }
    sq[0] = wave_sum(sq[0]);
    if (MT > 1) sq[1] = wave_sum(sq[1]);
    if (lane == 0) { stat[2 * wave] = sq[0]; stat[2 * wave + 1] = sq[1]; }
    __syncthreads();
    float rstd[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float t = 0.0f;
      for (int w = 0; w < S; ++w) t += stat[2 * w + j];
      rstd[j] = 1.0f / sqrtf(t / (float)a.k + a.eps);
    }
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int idx = lane + 64 * i;
      const float rr = rstd[MT > 1 && idx >= per_row ? 1 : 0];
      const float wv[8] = {nv[i][0].x, nv[i][0].y, nv[i][0].z, nv[i][0].w, nv[i][1].x, nv[i][1].y, nv[i][1].z, nv[i][1].w};
      uint32_t* vv = reinterpret_cast<uint32_t*>(&xv[i]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = round_bf16((bf16_bits_to_f32(vv[q] & 0xFFFFu) * rr) * wv[2 * q]);
        const float hi = round_bf16((bf16_bits_to_f32(vv[q] >> 16) * rr) * wv[2 * q + 1]);
        vv[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
      }
    }
  } else if (a.gnorm_w) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) gated_head_norm8(reinterpret_cast<uint32_t(&)[4]>(xv[i]), zv[i], nv[i][0], nv[i][1], a.gnorm_eps);
  }
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int idx = lane + 64 * i;
    if (idx < MT * per_row) {
      const int j = MT > 1 && idx >= per_row ? 1 : 0;
      uint4 v = xv[i];
      if constexpr (FMT == FMT_INT4) {        // (x0,x1)(x2,x3)(x4,x5)(x6,x7) → (x0,x4)(x1,x5)(x2,x6)(x3,x7)
        const uint32_t a0 = v.x, a1 = v.y, a2 = v.z, a3 = v.w;
        v.x = __builtin_amdgcn_perm(a2, a0, 0x05040100u);
        v.y = __builtin_amdgcn_perm(a2, a0, 0x07060302u);
        v.z = __builtin_amdgcn_perm(a3, a1, 0x05040100u);
        v.w = __builtin_amdgcn_perm(a3, a1, 0x07060302u);
      }
      *reinterpret_cast<uint4*>(xs + (size_t)j * ld + (idx - j * per_row) * 8) = v;
    }
  }
  wave_lds_sync();
  if constexpr (FMT == FMT_INT4) {
    // Σx over each (chunk, g, group) segment of 16 columns: steps {0,1} (group A) / {2,3} (group B) of k-group g
    for (int idx = lane; idx < MT * KW * 8; idx += 64) {
      const int j = idx / (KW * 8), rem = idx - j * KW * 8;
      const int cc = rem >> 3, g = (rem >> 1) & 3, gp = rem & 1;
      float sx = 0.0f;
      if (cc < kw) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const uint4 v = *reinterpret_cast<const uint4*>(xs + (size_t)j * ld + cc * 128 + 32 * (2 * gp + st) + 8 * g);
          const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) sx += bf16_bits_to_f32(vv[q] & 0xFFFFu) + bf16_bits_to_f32(vv[q] >> 16);
        }
      }
      seg[idx] = sx;
    }
    wave_lds_sync();
  }

  // ---- the slice's dot products, tile by tile --------------------------------------------------------------------
  const int g = lane >> 4, m_row = lane & 15;
  // tile jt from uu / ss; as soon as chunk cc is consumed, chunk cc of tile jn (the next, or jt itself at the last)
  // streams into its registers — a whole tile in flight with no second buffer
  auto tile_dot = [&](Units<FMT> (&uu)[KW], const uint4 (&ss)[NG], int jt, int jn, auto more) {
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    auto slice_chunk = [&](int cc) {
      const uint32_t dw[4] = {uu[cc].q.x, uu[cc].q.y, uu[cc].q.z, uu[cc].q.w};
      if constexpr (FMT == FMT_NVFP4) {
        uint4 xq[MT][4];
  #pragma unroll
        for (int t = 0; t < MT; ++t)
  #pragma unroll
          for (int s = 0; s < 4; ++s) xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * g + 8 * s);
        // chunk in its group: KW >= 8 slices start on a group, KW = 4 slices on one of its halves (c0 % 4 == 0)
        const uint4 pv = ss[KW >= 8 ? cc >> 3 : 0];
        const uint32_t word = KW >= 8 ? (cc & 6) == 0 ? pv.x : (cc & 6) == 2 ? pv.y : (cc & 6) == 4 ? pv.z : pv.w
                                      : (c0 & 4) ? (cc < 2 ? pv.z : pv.w) : (cc < 2 ? pv.x : pv.y);
        const f32x2 f = (cc & 1) ? __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true)
                                 : __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
        const uint32_t u0 = __float_as_uint(f.x), u1 = __float_as_uint(f.y);
        const float e[2] = {__uint_as_float(u0 & 0x7F800000u), __uint_as_float(u1 & 0x7F800000u)};
        const float mant[2] = {nv_mant(u0),
                               nv_mant(u1)};
  #pragma unroll
        for (int b = 0; b < 2; ++b) {
          float part[MT];
  #pragma unroll
          for (int t = 0; t < MT; ++t) part[t] = 0.0f;
  #pragma unroll
          for (int s = 2 * b; s < 2 * b + 2; ++s)
  #pragma unroll
            for (int j = 0; j < 4; ++j) {
              const bf16x2 w2 = cvt_fp4x2_bf16(dw[s], e[b], j);
  #pragma unroll
              for (int t = 0; t < MT; ++t) {
                const uint32_t xw = j == 0 ? xq[t][s].x : j == 1 ? xq[t][s].y : j == 2 ? xq[t][s].z : xq[t][s].w;
                part[t] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf16x2, xw), part[t], false);
              }
            }
  #pragma unroll
          for (int t = 0; t < MT; ++t) acc[t] = fmaf(part[t], mant[b], acc[t]);
        }
      } else if constexpr (FMT == FMT_INT4) {
        uint4 xq[MT][4];
        float sa[MT], sb[MT];
  #pragma unroll
        for (int t = 0; t < MT; ++t) {
  #pragma unroll
          for (int s = 0; s < 4; ++s) xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * s + 8 * g);
          sa[t] = seg[(t * KW + cc) * 8 + g * 2];
          sb[t] = seg[(t * KW + cc) * 8 + g * 2 + 1];
        }
        float d[2][MT];
  #pragma unroll
        for (int t = 0; t < MT; ++t) d[0][t] = d[1][t] = 0.0f;
  #pragma unroll
        for (int s = 0; s < 4; ++s)
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
        const float sca = bf16_bits_to_f32(uu[cc].sb.x & 0xFFFFu), bia = bf16_bits_to_f32(uu[cc].sb.x >> 16);
        const float scb = bf16_bits_to_f32(uu[cc].sb.y & 0xFFFFu), bib = bf16_bits_to_f32(uu[cc].sb.y >> 16);
  #pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[t] = fmaf(sca, fmaf(-128.0f, sa[t], d[0][t]), fmaf(bia, sa[t], acc[t]));
          acc[t] = fmaf(scb, fmaf(-128.0f, sb[t], d[1][t]), fmaf(bib, sb[t], acc[t]));
        }
      } else if constexpr (FMT == FMT_FP8) {
        uint4 xq[MT][2];                      // the lane's 16 columns 64·cc + 16·g + [0, 16)
      #pragma unroll
        for (int t = 0; t < MT; ++t)
      #pragma unroll
          for (int h = 0; h < 2; ++h) xq[t][h] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 64 + 16 * g + 8 * h);
      #pragma unroll
        for (int q = 0; q < 4; ++q)
      #pragma unroll
          for (int hi = 0; hi < 2; ++hi) {
            const bf16x2 w2 = cvt_fp8x2_bf16(dw[q], hi);   // columns 4q + 2hi, +1 of the lane's 16
      #pragma unroll
            for (int t = 0; t < MT; ++t) {
              const uint4 xv4 = xq[t][q >> 1];
              const int e = 2 * (q & 1) + hi;
              const uint32_t xw = e == 0 ? xv4.x : e == 1 ? xv4.y : e == 2 ? xv4.z : xv4.w;
              acc[t] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf16x2, xw), acc[t], false);
            }
          }
      } else {
        uint4 xq[MT];
  #pragma unroll
        for (int t = 0; t < MT; ++t) xq[t] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 32 + 8 * g);
  #pragma unroll
        for (int j = 0; j < 4; ++j)
  #pragma unroll
          for (int t = 0; t < MT; ++t) {
            const uint32_t xw = j == 0 ? xq[t].x : j == 1 ? xq[t].y : j == 2 ? xq[t].z : xq[t].w;
            acc[t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, dw[j]), __builtin_bit_cast(bf16x2, xw),
                                                     acc[t], false);
          }
      }
    };
#pragma unroll
    for (int cc = 0; cc < KW; ++cc) {
      if (cc < kw) slice_chunk(cc);
      if constexpr (decltype(more)::value) issue_chunk(uu, cc, jn);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float v = quad16_sum(acc[t]);
      if (g == 0) red[((jt * S + wave) * MT + t) * 16 + m_row] = v;
    }
  };
  // tiles in pairs, the scale pieces alternating between s0 and s1 (each loaded before the next tile's chunks). The
  // last tile issues nothing after it: a load left in flight there is waited for where its registers are reused (a
  // round trip on every wave's way out), so whether a call site issues the next tile is fixed at compile time.
  using Issue = std::true_type;
  using NoIssue = std::false_type;
  int j = 0;
  for (; j + 2 < ntl; j += 2) {
    issue_scales(s1, j + 1);
    tile_dot(u0, s0, j, j + 1, Issue{});
    issue_scales(s0, j + 2);
    tile_dot(u0, s1, j + 1, j + 2, Issue{});
  }
  if (j + 1 < ntl) {
    issue_scales(s1, j + 1);
    tile_dot(u0, s0, j, j + 1, Issue{});
    tile_dot(u0, s1, j + 1, j + 1, NoIssue{});
  } else {
    tile_dot(u0, s0, j, j, NoIssue{});
  }

  // ---- per tile: the K slices in wave order, then the epilogue (16-lane groups hold one tile's rows) -----------
  __syncthreads();
  if (wave != 0) return;
  const int total = ntl * MT * 16;
  for (int base = 0; base < total; base += 64) {
    const int idx = base + threadIdx.x;
    const bool ok = idx < total;
    const int q = ok ? idx >> 4 : 0, r = idx & 15;
    const int jt = q / MT, t = q - jt * MT;
    float v = slice_sum_lane(red + (jt * S * MT + t) * 16, MT * 16, S, r);
    const int tile = tile_of(jt);
    const int row = tile * 16 + r;
    if (a.ks > 1) {                             // this split's partial; gemv_tk_reduce adds the splits in order
      if (ok && t < cnt) a.part[((long long)split * a.m + t) * a.n_tiles * 16 + row] = v;
      continue;
    }
    v *= a.row_scale != nullptr ? a.row_scale[(long long)expert * a.n_tiles * 16 + row] : 1.0f;
    const float up = __shfl_down(v, 8, 16);
    if (ok) emit(a, epilogue_of(a, expert), pairs, cnt, tile, true, r, t, v, up);
  }
}

// ---- gemv_rowm: 3 <= M <= 16, NVFP4, FP8 and INT4 ---------------------------------------------------------------
// The gemv_row wave layout on the matrix cores, over several tiles per workgroup. Workgroup = S waves over tiles
// blockIdx.x + j·G (j < ntl) and K split blockIdx.z; wave w owns a 512-column slice (4 NVFP4 / 8 FP8 chunks) of
// every one of them. The
// wave's activations for those chunks stay in VGPRs for the whole launch as the F16 A operands of
// v_mfma_f32_16x16x32_f16 (token = A row; each token power-of-two scaled into F16 range over the wave's slice;
// normalized first when the input norm is fused); the weights are the B operand, decoded exactly to F16. Each wave
// keeps two tiles in flight (NVFP4 / FP8; one for INT4) and issues the next as soon as one is consumed. A
// tile's K slices meet in LDS after the last tile, in the gemv_row order. INT4: the codes decode to exact F16
// integers, the activations take the codes' column order (int4_perm8) and each 64-column group's dot product is
// scaled and offset by its (scale, bias) pair with the token's Σx over the group (held per lane for the launch).
// LDS: nw[K] (fused norm) | stat[S][16] | red[rt][S][16 tokens][16 rows].
template <int FMT>
__global__ __launch_bounds__(768) void gemv_rowm(Args a) {
  constexpr int KC = chunk_cols(FMT), KW = 512 / KC;   // a wave's slice is 512 columns: 4 NVFP4 / INT4, 8 FP8 chunks
  constexpr int SPC = KC / 32;                  // MFMA steps per chunk: the lane's KC/4 columns, 8 per step
  static_assert(FMT == FMT_NVFP4 || FMT == FMT_FP8 || FMT == FMT_INT4, "gemv_rowm: NVFP4, FP8 or INT4");
  constexpr bool I4 = FMT == FMT_INT4;
  constexpr int UB = I4 ? UNIT_Q : 1024;        // bytes from one chunk's codes to the next
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const int G = gridDim.x;
  const int ntl = (a.n_tiles - 1 - (int)blockIdx.x) / G + 1;
  const int cnt = a.m;
  const int split = blockIdx.z;
  const int c0_raw = split * a.kc + wave * KW;
  const bool active = c0_raw < min(a.chunks, (split + 1) * a.kc);
  const int c0 = active ? c0_raw : 0;
  const int kw = active ? min(KW, min(a.chunks, (split + 1) * a.kc) - c0) : 0;   // chunks this wave holds (≤ KW)
  const int g = lane >> 4, m_row = lane & 15;
  const uint8_t* wmat = a.w;
  auto tile_of = [&](int j) { return (int)blockIdx.x + j * G; };
  float* nws = reinterpret_cast<float*>(smem);                                  // [K] when the norm is fused
  float* stat = nws + (a.norm_w ? a.k : 0);                                    // [S][16]
  float* sxl = stat + S * 16;                                                  // INT4: [S][KW][2][16]
  float* red = sxl + (I4 ? S * KW * 2 * 16 : 0);                               // [rt][S][16][16]

  // ---- the first tile's weights, then the activations ------------------------------------------------------------
  const long long c0_off = FMT == FMT_NVFP4 ? nv_code_off(c0) : (long long)c0 * unit_bytes(FMT);
  // NVFP4 / FP8 keep two tiles in flight per wave (the 12-wave workgroup leaves 168 VGPRs a lane); INT4's Σx
  // terms leave room for one
  constexpr int DEPTH = I4 ? 1 : 2;
  uint2 sb0[I4 ? KW : 1], sb1[I4 ? KW : 1];     // INT4: the (scale, bias) pairs of row m_row's two groups per chunk
  auto issue = [&](uint4 (&u)[KW], uint4& sv, uint2 (&sb)[I4 ? KW : 1], int j) {
    const uint8_t* tbase = wmat + (long long)tile_of(j) * a.tile_stride;
    // every load unconditional (a chunk past the wave's kw re-reads chunk 0 and is never used), so the loads of
    // the tiles in flight stay in issue order and a tile waits for its own loads only
    if constexpr (FMT == FMT_NVFP4) {
      const int gi = c0 >> 3;
      const uint8_t* p = tbase + nv_scale_off(gi, a.chunks);
      // 16 scale bytes a lane in a group of 8 chunks, else 8 (a group of at most 4 chunks starts a slice, so its
      // lanes use sv.x / sv.y only and t1 repeats t0)
      const bool wide = nv_piece(nv_group_chunks(gi, a.chunks)) == 16;
      const uint2 t0 = *reinterpret_cast<const uint2*>(p + (wide ? 16 : 8) * lane);
      const uint2 t1 = *reinterpret_cast<const uint2*>(p + (wide ? 16 * lane + 8 : 8 * lane));
      sv = uint4{t0.x, t0.y, t1.x, t1.y};
    } else {
      sv = uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int cc = 0; cc < KW; ++cc) {           // 1 KiB of codes per chunk
      const long long off = c0_off + (cc < kw ? cc : 0) * UB;
      u[cc] = ld_stream(tbase + off + 16 * lane);
      if constexpr (I4) sb[cc] = *reinterpret_cast<const uint2*>(tbase + off + 1024 + 8 * (lane & 15));
    }
    __builtin_amdgcn_sched_barrier(0);          // the tile's loads stay where they are in the issue order
  };
  uint4 u0[KW], s0, u1[KW], s1;
  issue(u0, s0, sb0, 0);
  if (DEPTH > 1) issue(u1, s1, sb1, min(1, ntl - 1));

  // x[token m_row][c0·KC + cc·KC + col(g, s) + (0..7)]: the A operand of step s of chunk cc, col(g, s) =
  // (KC/4)·g + 8s (NVFP4 / FP8) or 32s + 8g (INT4: the codes' column order in a unit)
  const bool real = m_row < cnt;
  auto xcol = [&](int s) { return I4 ? 32 * s + 8 * g : (KC / 4) * g + 8 * s; };
  uint4 xa[KW][SPC];
  const uint16_t* xrow = a.x + (long long)(real ? m_row : 0) * a.ldx + c0 * KC;
#pragma unroll
  for (int cc = 0; cc < KW; ++cc)
#pragma unroll
    for (int s = 0; s < SPC; ++s)
      xa[cc][s] = cc < kw ? *reinterpret_cast<const uint4*>(xrow + cc * KC + xcol(s)) : uint4{0u, 0u, 0u, 0u};
  if (!real) {                                // padding token rows: zero operands (their loads read row 0)
#pragma unroll
    for (int cc = 0; cc < KW; ++cc)
#pragma unroll
      for (int s = 0; s < SPC; ++s) xa[cc][s] = uint4{0u, 0u, 0u, 0u};
  }

  if (a.norm_w) {
    // the norm weights into LDS once; Σx² per token over the row from every wave's slice
    for (int i = threadIdx.x; i < a.k / 4; i += blockDim.x)
      reinterpret_cast<float4*>(nws)[i] = reinterpret_cast<const float4*>(a.norm_w)[i];
    float sq = 0.0f;
#pragma unroll
    for (int cc = 0; cc < KW; ++cc)
#pragma unroll
      for (int s = 0; s < SPC; ++s) {
        const uint32_t vv[4] = {xa[cc][s].x, xa[cc][s].y, xa[cc][s].z, xa[cc][s].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)           // x0² + x1² straight from the BF16 pair: no FP32 copies of the slice
          sq = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, vv[q]), __builtin_bit_cast(bf16x2, vv[q]), sq, false);
      }
    sq = add_xor32(add_xor16(active ? sq : 0.0f));    // the four lanes of token m_row
    if (g == 0) stat[wave * 16 + m_row] = sq;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < S; ++w) t += stat[w * 16 + m_row];
    const float rr = 1.0f / sqrtf(t / (float)a.k + a.eps);
#pragma unroll
    for (int cc = 0; cc < KW; ++cc)
#pragma unroll
      for (int s = 0; s < SPC; ++s) {
        if (cc >= kw) break;
        const float* wv = nws + (c0 + cc) * KC + xcol(s);
        const float4 w0 = *reinterpret_cast<const float4*>(wv), w1 = *reinterpret_cast<const float4*>(wv + 4);
        const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        uint32_t* vv = reinterpret_cast<uint32_t*>(&xa[cc][s]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = round_bf16((bf16_bits_to_f32(vv[q] & 0xFFFFu) * rr) * ww[2 * q]);
          const float hi = round_bf16((bf16_bits_to_f32(vv[q] >> 16) * rr) * ww[2 * q + 1]);
          vv[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
        }
        __builtin_amdgcn_sched_barrier(0);    // one step's weights at a time (the operands already hold 64 VGPRs)
      }
  }
  // F16 operands: per token, 2^-p brings the slice max into [2^14, 2^15) (exact within 2^28 of the max). The max
  // is taken on the BF16 magnitudes as integers (same order for finite values), so no FP32 copy of the slice exists.
  uint32_t mb = 0;
#pragma unroll
  for (int cc = 0; cc < KW; ++cc)
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
      const uint32_t vv[4] = {xa[cc][s].x, xa[cc][s].y, xa[cc][s].z, xa[cc][s].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) mb = max(mb, max(vv[q] & 0x7FFFu, (vv[q] >> 16) & 0x7FFFu));
    }
  float mx = bf16_bits_to_f32(mb);
  mx = max_xor32(max_xor16(mx));
  const int pe = mx == 0.0f ? 0 : (int)((__float_as_uint(mx) >> 23) & 0xFF) - 127 - 14;
  const float inv = __uint_as_float((uint32_t)(127 - pe) << 23);
  const float psc = __uint_as_float((uint32_t)(127 + pe) << 23);
#pragma unroll
  for (int cc = 0; cc < KW; ++cc)             // in place: xa now holds the F16 operands
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
      uint32_t* vv = reinterpret_cast<uint32_t*>(&xa[cc][s]);
      if constexpr (I4) {                     // element e of the operand = column int4_perm8(e)
        uint16_t hv[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) { hv[2 * q] = vv[q] & 0xFFFFu; hv[2 * q + 1] = vv[q] >> 16; }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f16x2 h = {(f16_t)(bf16_bits_to_f32(hv[int4_perm8(2 * q)]) * inv),
                           (f16_t)(bf16_bits_to_f32(hv[int4_perm8(2 * q + 1)]) * inv)};
          vv[q] = __builtin_bit_cast(uint32_t, h);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f16x2 h = {(f16_t)(bf16_bits_to_f32(vv[q] & 0xFFFFu) * inv), (f16_t)(bf16_bits_to_f32(vv[q] >> 16) * inv)};
          vv[q] = __builtin_bit_cast(uint32_t, h);
        }
      }
      __builtin_amdgcn_sched_barrier(0);      // one operand at a time: no FP32 copies of the whole slice
    }
  // the output rows of lane l are tokens 4g + i: their scales from the lanes that hold those tokens' A rows
  float ps[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ps[i] = __shfl(psc, 4 * g + i, 64);
  // INT4: Σx (prescaled F16) per 64-column group — steps {0, 1} and {2, 3} of each chunk — per token (the sum over
  // its four k-group lanes), kept in the wave's LDS rows: tile_mma reads those of its output tokens 4g + i
  float* sxw = sxl + wave * KW * 2 * 16;
  if constexpr (I4) {
#pragma unroll
    for (int cc = 0; cc < KW; ++cc)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        float sx = 0.0f;
#pragma unroll
        for (int s = 2 * gp; s < 2 * gp + 2; ++s) {
          const f16x8 h = __builtin_bit_cast(f16x8, xa[cc][s]);
#pragma unroll
          for (int e = 0; e < 8; ++e) sx += (float)h[e];
        }
        sx = add_xor32(add_xor16(cc < kw ? sx : 0.0f));
        if (g == 0) sxw[(cc * 2 + gp) * 16 + m_row] = sx;
      }
    wave_lds_sync();
  }

  // ---- tile by tile: 16 MFMAs over the slice, the partial (tokens × rows) into LDS ----------------------------------
  auto tile_mma = [&](const uint4 (&u)[KW], const uint4 sv, const uint2 (&sbs)[I4 ? KW : 1], int jt) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < KW; ++cc) {
      if (cc >= kw) break;
      const uint32_t dw[4] = {u[cc].x, u[cc].y, u[cc].z, u[cc].w};
      if constexpr (FMT == FMT_NVFP4) {
        const uint32_t word = (c0 & 4) ? (cc < 2 ? sv.z : sv.w) : (cc < 2 ? sv.x : sv.y);
        const f32x2 f = (cc & 1) ? __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true)
                                 : __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
        const uint32_t b0 = __float_as_uint(f.x), b1 = __float_as_uint(f.y);
        const float e0 = __uint_as_float(b0 & 0x7F800000u), e1 = __uint_as_float(b1 & 0x7F800000u);
        const f16_t m0 = (f16_t)nv_mant(b0);
        const f16_t m1 = (f16_t)nv_mant(b1);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const f16x8 bv = nvfp4_decode8(dw[s], s < 2 ? e0 : e1, s < 2 ? m0 : m1);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xa[cc][s]), bv, acc, 0, 0, 0);
        }
      } else if constexpr (I4) {                // the two 64-column groups, each scaled and offset on its own
        f32x4 da = {0.f, 0.f, 0.f, 0.f}, db = {0.f, 0.f, 0.f, 0.f};
        da = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xa[cc][0]), int4_decode8(dw[0]), da, 0, 0, 0);
        da = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xa[cc][1]), int4_decode8(dw[1]), da, 0, 0, 0);
        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xa[cc][2]), int4_decode8(dw[2]), db, 0, 0, 0);
        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xa[cc][3]), int4_decode8(dw[3]), db, 0, 0, 0);
        const uint2 sb = sbs[cc];
        const float sca = bf16_bits_to_f32(sb.x & 0xFFFFu), bia = bf16_bits_to_f32(sb.x >> 16);
        const float scb = bf16_bits_to_f32(sb.y & 0xFFFFu), bib = bf16_bits_to_f32(sb.y >> 16);
        const f32x4 sxa = *reinterpret_cast<const f32x4*>(sxw + (cc * 2) * 16 + 4 * g);
        const f32x4 sxb = *reinterpret_cast<const f32x4*>(sxw + (cc * 2 + 1) * 16 + 4 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i] = fmaf(sca, da[i], fmaf(bia, sxa[i], acc[i]));
          acc[i] = fmaf(scb, db[i], fmaf(bib, sxb[i], acc[i]));
        }
      } else {                                  // FP8: the lane's 16 codes, 8 per step
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const f16x8 bv = fp8_decode8(dw[2 * s], dw[2 * s + 1]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xa[cc][s]), bv, acc, 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);      // decode chunk by chunk: keeps the decoded operands' registers few
    }
    float* rp = red + ((jt * S + wave) * 16) * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) rp[(4 * g + i) * 16 + m_row] = active ? acc[i] * ps[i] : 0.0f;
  };
  if constexpr (DEPTH == 1) {
    for (int j = 0; j < ntl; ++j) {
      tile_mma(u0, s0, sb0, j);
      if (j + 1 < ntl) issue(u0, s0, sb0, j + 1);
    }
  } else {
    // tiles j and j + 1 in flight: consume one, issue j + 2 into its place, so each tile's loads are older than
    // exactly one tile's and its wait leaves the other tile in flight. No issue past the last tile: a load left in
    // flight there is waited for where its registers are reused (a round trip on every wave's way out), so the
    // tail's call sites are spelled out.
    int j = 0;
    if constexpr (FMT == FMT_FP8) {             // the longer FP8 decode: the spelled-out tail spills (40 B / lane)
      for (; j + 1 < ntl; j += 2) {
        tile_mma(u0, s0, sb0, j);
        issue(u0, s0, sb0, min(j + 2, ntl - 1));
        tile_mma(u1, s1, sb1, j + 1);
        issue(u1, s1, sb1, min(j + 3, ntl - 1));
      }
      if (j < ntl) tile_mma(u0, s0, sb0, j);
    } else {
    for (; j + 3 < ntl; j += 2) {
      tile_mma(u0, s0, sb0, j);
      issue(u0, s0, sb0, j + 2);
      tile_mma(u1, s1, sb1, j + 1);
      issue(u1, s1, sb1, j + 3);
    }
    if (j + 2 < ntl) {                          // three left: j, j + 1 in flight, j + 2 still to issue
      tile_mma(u0, s0, sb0, j);
      issue(u0, s0, sb0, j + 2);
      tile_mma(u1, s1, sb1, j + 1);
      tile_mma(u0, s0, sb0, j + 2);
    } else if (j + 1 < ntl) {
      tile_mma(u0, s0, sb0, j);
      tile_mma(u1, s1, sb1, j + 1);
    } else {
      tile_mma(u0, s0, sb0, j);
    }
    }
  }

  // ---- per (tile, token): the K slices in the gemv_row order, then the epilogue --------------------------------
  __syncthreads();
  for (int pi = wave; pi < ntl * cnt; pi += S) {
    const int jt = pi / cnt, t = pi - jt * cnt;
    const int tile = tile_of(jt);
    float v = slice_sum(red + (jt * S * 16 + t) * 16, 16 * 16, S, lane);
    const int row = tile * 16 + m_row;
    if (a.ks > 1) {
      if (g == 0) a.part[((long long)split * a.m + t) * a.n_tiles * 16 + row] = v;
      continue;
    }
    v *= a.row_scale != nullptr ? a.row_scale[row] : 1.0f;
    const float up = __shfl_down(v, 8, 16);
    if (g == 0) emit(a, a.epilogue, nullptr, cnt, tile, true, m_row, t, v, up);
  }
}

// ---- the tile × K-split kernel ----------------------------------------------------------------------------------
// Work item: (group of TB consecutive 16-row tiles, K split s = chunks [s·kc, min(chunks, (s+1)·kc))). A workgroup
// of S waves stages the split's activations once — BF16 for the VALU path (M <= 2), per-token power-of-two
// prescaled F16 for MFMA (M <= 16) — and wave w takes tiles w, w + S, … of the group over the whole split, streaming
// its units through a D-deep register ring that runs on across tile boundaries. Every tile ends in the wave that
// computed it: with one split the epilogue runs from its registers; with several the wave writes FP32 partials and
// gemv_tk_reduce adds them in split order (deterministic). The activations are read once per workgroup, so the
// L2 traffic they cost is (workgroups × split width) rather than (tiles × K) — the difference between the two at
// M = 8 is several times the weight bytes.
// LDS: xs[rows][kw·KC + 8] | pscale[16] (MFMA) | (INT4) seg / gsum.
template <int FMT, int MT, int D, bool PIECES>
__global__ __launch_bounds__(512) void gemv_tk(Args a) {
  constexpr bool MF = MT > 2;
  constexpr int KC = chunk_cols(FMT);
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (scalar) in the compiler's view
  const int S = blockDim.x >> 6;
  const int split = blockIdx.y;
  int expert = 0, cnt = a.m;
  const int32_t* pairs = nullptr;
  if (a.groups) {
    const int32_t* g = a.groups + blockIdx.z * GROUP_REC;
    expert = g[0];
    cnt = g[1];
    pairs = g + 2;
    if (cnt <= 0 || expert < 0) return;       // the whole workgroup leaves together
  }
  if (cnt > MT) cnt = MT;
  auto xrow_of = [&](int j) -> long long {
    if (!pairs) return j;
    const int p = pairs[j];
    return a.x_per_slot ? p : p / a.top_k;
  };
  const int kb = split * a.kc;
  const int kw = min(a.chunks, kb + a.kc) - kb;
  const int cols = kw * KC;
  const int ld = cols + 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  const int xrows = cnt;
  float* pscale = reinterpret_cast<float*>(smem + (size_t)a.lds_rows * ld * 2);   // [16]
  float* extra = pscale + 16;                                             // INT4: seg [MT][kw][8] / gsum [kw·2][16]
  const uint8_t* zero = reinterpret_cast<const uint8_t*>(extra + (FMT == FMT_INT4 ? (MF ? kw * 2 * 16 : MT * kw * 8) : 0));

  // ---- this wave's tiles and the ring: the weights start streaming before anything else ---------------------
  const int tile0 = blockIdx.x * a.tb;
  const int ntl = min(a.tb, a.n_tiles - tile0);
  const int nt_w = ntl > wave ? (ntl - wave + S - 1) / S : 0;   // tiles wave, wave + S, … < ntl
  const int total = nt_w * kw;
  const uint8_t* wmat = a.w + (long long)expert * a.expert_stride;
  int lt = 0, lc = 0, left = total;
  // NVFP4 block scales (PIECES): one 16-byte piece per group of 8 chunks. The split width is a multiple of 8, so
  // every 8th unit of the stream starts a group; the stream runs in steps of 16 units with the ring (D = 8) and a
  // 2-slot piece ring both indexed statically. Without PIECES each unit brings its two scale bytes itself.
  uint4 spc[2] = {uint4{0u, 0u, 0u, 0u}, uint4{0u, 0u, 0u, 0u}};
  auto load_next = [&](Units<FMT>& u) {
    load_chunk<FMT, !PIECES>(u, wmat + (long long)(tile0 + wave + lt * S) * a.tile_stride, kb + lc, a.chunks, lane);
    if (left > 1) {
      --left;
      if (++lc == kw) { lc = 0; ++lt; }
    }
  };
  auto piece_of = [&](const uint8_t* tb, int c) {
    const int gi = c >> 3;
    const uint8_t* pp = tb + nv_scale_off(gi, a.chunks);
    return *reinterpret_cast<const uint4*>(pp + 16 * lane);
  };
  Units<FMT> ring[D];
  if (total > 0) {
    if constexpr (PIECES) spc[0] = piece_of(wmat + (long long)(tile0 + wave) * a.tile_stride, kb);
#pragma unroll
    for (int i = 0; i < D; ++i) load_next(ring[i]);
  }

  // ---- stage the split's activations: wave j stages token rows j, j + S, … -------------------------------------
  if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(const_cast<uint8_t*>(zero))[threadIdx.x] = 0u;
  // the epilogue's inputs staged once, behind the ring's first units: the row scales of the workgroup's tiles and
  // the group's pair ids — a global load inside the stream would wait for every unit of the ring issued before it
  float* rs_s = reinterpret_cast<float*>(const_cast<uint8_t*>(zero) + 64);   // [tb·16]
  int* pairs_s = reinterpret_cast<int*>(rs_s + a.tb * 16);                   // [16]
  const int n_pad = a.n_tiles * 16;
  for (int i = threadIdx.x; i < ntl * 16; i += blockDim.x)
    rs_s[i] = a.row_scale != nullptr ? a.row_scale[(long long)expert * n_pad + tile0 * 16 + i] : 1.0f;
  if (pairs && (int)threadIdx.x < cnt) pairs_s[threadIdx.x] = pairs[threadIdx.x];
  for (int j = wave; j < xrows; j += S) {
    const uint16_t* src = a.x + xrow_of(j) * a.ldx + kb * KC;
    uint16_t* dst = xs + (size_t)j * ld;
    const int nv = cols / 8;
    float sq = 0.0f;
    const bool whole = kw == a.chunks;          // the split covers the row: its sum of squares comes with the staging
    for (int v = lane; v < nv; v += 64) {
      const uint4 q = *reinterpret_cast<const uint4*>(src + v * 8);
      if (a.norm_w && whole) {
        const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16_bits_to_f32(qq[i] & 0xFFFFu), hi = bf16_bits_to_f32(qq[i] >> 16);
          sq = fmaf(lo, lo, fmaf(hi, hi, sq));
        }
      }
      *reinterpret_cast<uint4*>(dst + v * 8) = q;
    }
    if (a.norm_w && !whole) {                   // K split: the whole row's sum of squares, in the same order
      const uint16_t* row = a.x + xrow_of(j) * a.ldx;
      for (int v = lane; v < a.chunks * KC / 8; v += 64) {
        const uint4 q = *reinterpret_cast<const uint4*>(row + v * 8);
        const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16_bits_to_f32(qq[i] & 0xFFFFu), hi = bf16_bits_to_f32(qq[i] >> 16);
          sq = fmaf(lo, lo, fmaf(hi, hi, sq));
        }
      }
    }
    float rr = 1.0f;
    if (a.norm_w) rr = 1.0f / sqrtf(wave_sum(sq) / (float)a.k + a.eps);
    float mx = 0.0f;
    if (a.norm_w || a.gnorm_w || MF || FMT == FMT_INT4) {
      wave_lds_sync();
      for (int v = lane; v < nv; v += 64) {      // nv is a multiple of 16: whole 16-lane rows stay active
        uint4 q = *reinterpret_cast<const uint4*>(dst + v * 8);
        uint32_t* qq = reinterpret_cast<uint32_t*>(&q);
        if (a.gnorm_w) {
          const int col = kb * KC + v * 8;
          const uint4 zv = *reinterpret_cast<const uint4*>(a.gnorm_z + xrow_of(j) * a.ld_gnorm_z + col);
          const float4 w0 = *reinterpret_cast<const float4*>(a.gnorm_w + (col & 127));
          const float4 w1 = *reinterpret_cast<const float4*>(a.gnorm_w + (col & 127) + 4);
          gated_head_norm8(reinterpret_cast<uint32_t(&)[4]>(q), zv, w0, w1, a.gnorm_eps);
        }
        if (a.norm_w) {
          const int col = kb * KC + v * 8;
          const float4 w0 = *reinterpret_cast<const float4*>(a.norm_w + col);
          const float4 w1 = *reinterpret_cast<const float4*>(a.norm_w + col + 4);
          const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float lo = round_bf16((bf16_bits_to_f32(qq[i] & 0xFFFFu) * rr) * wv[2 * i]);
            const float hi = round_bf16((bf16_bits_to_f32(qq[i] >> 16) * rr) * wv[2 * i + 1]);
            qq[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
          }
        }
        if (MF) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            mx = fmaxf(mx, fmaxf(fabsf(bf16_bits_to_f32(qq[i] & 0xFFFFu)), fabsf(bf16_bits_to_f32(qq[i] >> 16))));
        }
        if (!MF && FMT == FMT_INT4) {       // (x0,x1)(x2,x3)(x4,x5)(x6,x7) → (x0,x4)(x1,x5)(x2,x6)(x3,x7)
          const uint32_t a0 = qq[0], a1 = qq[1], a2 = qq[2], a3 = qq[3];
          qq[0] = __builtin_amdgcn_perm(a2, a0, 0x05040100u);
          qq[1] = __builtin_amdgcn_perm(a2, a0, 0x07060302u);
          qq[2] = __builtin_amdgcn_perm(a3, a1, 0x05040100u);
          qq[3] = __builtin_amdgcn_perm(a3, a1, 0x07060302u);
        }
        *reinterpret_cast<uint4*>(dst + v * 8) = q;
      }
    }
    if constexpr (MF && FMT == FMT_BF16) {
      if (lane == 0) pscale[j] = 1.0f;                // BF16 weights: the MFMA takes the BF16 activations as they are
    } else if constexpr (MF) {
      // F16 operands: 2^-p brings the row max into [2^14, 2^15) (exact for everything within 2^28 of the max)
      mx = wave_max(mx);
      const int p = mx == 0.0f ? 0 : (int)((__float_as_uint(mx) >> 23) & 0xFF) - 127 - 14;
      const float inv = __uint_as_float((uint32_t)(127 - p) << 23);
      if (lane == 0) pscale[j] = __uint_as_float((uint32_t)(127 + p) << 23);
      wave_lds_sync();
      for (int v = lane; v < nv; v += 64) {
        const uint4 q = *reinterpret_cast<const uint4*>(dst + v * 8);
        const uint16_t* hv = reinterpret_cast<const uint16_t*>(&q);
        f16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (f16_t)(bf16_bits_to_f32(hv[FMT == FMT_INT4 ? int4_perm8(i) : i]) * inv);
        *reinterpret_cast<f16x8*>(dst + v * 8) = o;
      }
    }
    wave_lds_sync();
    if constexpr (FMT == FMT_INT4) {
      if constexpr (MF) {
        // Σx (prescaled F16) per 64 columns: the bias term of the affine groups
        for (int gi = lane; gi < kw * 2; gi += 64) {
          const f16_t* px = reinterpret_cast<const f16_t*>(dst + gi * 64);
          float sx = 0.0f;
          for (int i = 0; i < 64; ++i) sx += (float)px[i];
          extra[gi * 16 + j] = sx;
        }
      } else {
        // Σx over each (chunk, g, group) segment of 16 columns: steps {0,1} (group A) / {2,3} (group B) of k-group g
        for (int idx = lane; idx < kw * 8; idx += 64) {
          const int cc = idx >> 3, g = (idx >> 1) & 3, gp = idx & 1;
          float sx = 0.0f;
#pragma unroll
          for (int st = 0; st < 2; ++st) {
            const uint4 v = *reinterpret_cast<const uint4*>(dst + cc * 128 + 32 * (2 * gp + st) + 8 * g);
            const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) sx += bf16_bits_to_f32(vv[q] & 0xFFFFu) + bf16_bits_to_f32(vv[q] >> 16);
          }
          extra[(j * kw + cc) * 8 + g * 2 + gp] = sx;
        }
      }
    }
  }
  if constexpr (MF && FMT == FMT_INT4) {   // padding token rows: zero sums
    for (int idx = threadIdx.x; idx < kw * 2 * 16; idx += blockDim.x)
      if ((idx & 15) >= xrows) extra[idx] = 0.0f;
  }
  __syncthreads();

  const int g = lane >> 4, m_row = lane & 15;
  // MFMA: A row = token m_row (a padding token reads the 16 zero bytes at every step)
  const bool a_real = m_row < cnt;
  const uint8_t* a_row = a_real ? reinterpret_cast<const uint8_t*>(xs + (size_t)m_row * ld) : zero;
  const int a_mask = a_real ? ~0 : 0;

  float acc_v[MT > 2 ? 1 : MT];
  f32x4 acc_m = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < (MT > 2 ? 1 : MT); ++t) acc_v[t] = 0.0f;

  auto compute = [&](const Units<FMT>& u, int cc, int par, uint32_t s_unit) {
    if constexpr (MF) {
      const int kl = cc * KC;
      if constexpr (FMT == FMT_BF16) {
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(a_row + (((kl + 8 * g) * 2) & a_mask));
        union { uint4 u; bf16x8 b; } wv;
        wv.u = u.q;
        acc_m = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, wv.b, acc_m, 0, 0, 0);
      } else if constexpr (FMT == FMT_NVFP4) {
        f16x8 av[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) av[s] = *reinterpret_cast<const f16x8*>(a_row + (((kl + 32 * g + 8 * s) * 2) & a_mask));
        uint32_t two = s_unit;
        if constexpr (PIECES) {
          const uint4 pv = spc[par];
          const int ci = cc & 7;
          const uint32_t word = (ci >> 1) == 0 ? pv.x : (ci >> 1) == 1 ? pv.y : (ci >> 1) == 2 ? pv.z : pv.w;
          two = (ci & 1) ? word >> 16 : word & 0xFFFFu;
        }
        const ScalePair sp = nvfp4_scales(two);
        const uint32_t dw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const f16x8 bv = nvfp4_decode8(dw[s], s < 2 ? sp.e0 : sp.e1, s < 2 ? sp.m0 : sp.m1);
          acc_m = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[s], bv, acc_m, 0, 0, 0);
        }
      } else {
        f16x8 av[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) av[s] = *reinterpret_cast<const f16x8*>(a_row + (((kl + 32 * s + 8 * g) * 2) & a_mask));
        const f32x4 sxa = *reinterpret_cast<const f32x4*>(extra + (cc * 2) * 16 + 4 * g);
        const f32x4 sxb = *reinterpret_cast<const f32x4*>(extra + (cc * 2 + 1) * 16 + 4 * g);
        const uint32_t dw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
        f32x4 da = {0.f, 0.f, 0.f, 0.f}, db = {0.f, 0.f, 0.f, 0.f};
        da = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[0], int4_decode8(dw[0]), da, 0, 0, 0);
        da = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[1], int4_decode8(dw[1]), da, 0, 0, 0);
        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[2], int4_decode8(dw[2]), db, 0, 0, 0);
        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[3], int4_decode8(dw[3]), db, 0, 0, 0);
        const float sca = bf16_bits_to_f32(u.sb.x & 0xFFFFu), bia = bf16_bits_to_f32(u.sb.x >> 16);
        const float scb = bf16_bits_to_f32(u.sb.y & 0xFFFFu), bib = bf16_bits_to_f32(u.sb.y >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc_m[i] = fmaf(sca, da[i], fmaf(bia, sxa[i], acc_m[i]));
          acc_m[i] = fmaf(scb, db[i], fmaf(bib, sxb[i], acc_m[i]));
        }
      }
    } else if constexpr (FMT == FMT_NVFP4) {
      uint4 xq[MT][4];
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * g + 8 * s);
      uint32_t two = s_unit;
      if constexpr (PIECES) {
        const uint4 pv = spc[par];
        const int ci = cc & 7;
        const uint32_t word = (ci >> 1) == 0 ? pv.x : (ci >> 1) == 1 ? pv.y : (ci >> 1) == 2 ? pv.z : pv.w;
        two = (ci & 1) ? word >> 16 : word & 0xFFFFu;
      }
      const f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)two, false);
      const uint32_t u0 = __float_as_uint(f.x), u1 = __float_as_uint(f.y);
      const float e[2] = {__uint_as_float(u0 & 0x7F800000u), __uint_as_float(u1 & 0x7F800000u)};
      const float mant[2] = {nv_mant(u0),
                             nv_mant(u1)};
      const uint32_t dw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float part[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) part[t] = 0.0f;
#pragma unroll
        for (int s = 2 * b; s < 2 * b + 2; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x2 w2 = cvt_fp4x2_bf16(dw[s], e[b], j);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
              const uint32_t xw = j == 0 ? xq[t][s].x : j == 1 ? xq[t][s].y : j == 2 ? xq[t][s].z : xq[t][s].w;
              part[t] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf16x2, xw), part[t], false);
            }
          }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc_v[t] = fmaf(part[t], mant[b], acc_v[t]);
      }
    } else if constexpr (FMT == FMT_INT4) {
      uint4 xq[MT][4];
      float sa[MT], sb[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int s = 0; s < 4; ++s) xq[t][s] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 128 + 32 * s + 8 * g);
        sa[t] = extra[(t * kw + cc) * 8 + g * 2];
        sb[t] = extra[(t * kw + cc) * 8 + g * 2 + 1];
      }
      const uint32_t dw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
      float d[2][MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) d[0][t] = d[1][t] = 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
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
      const float sca = bf16_bits_to_f32(u.sb.x & 0xFFFFu), bia = bf16_bits_to_f32(u.sb.x >> 16);
      const float scb = bf16_bits_to_f32(u.sb.y & 0xFFFFu), bib = bf16_bits_to_f32(u.sb.y >> 16);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        acc_v[t] = fmaf(sca, fmaf(-128.0f, sa[t], d[0][t]), fmaf(bia, sa[t], acc_v[t]));
        acc_v[t] = fmaf(scb, fmaf(-128.0f, sb[t], d[1][t]), fmaf(bib, sb[t], acc_v[t]));
      }
    } else {
      uint4 xq[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) xq[t] = *reinterpret_cast<const uint4*>(xs + (size_t)t * ld + cc * 32 + 8 * g);
      const uint32_t dw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint32_t xw = j == 0 ? xq[t].x : j == 1 ? xq[t].y : j == 2 ? xq[t].z : xq[t].w;
          acc_v[t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, dw[j]), __builtin_bit_cast(bf16x2, xw),
                                                     acc_v[t], false);
        }
    }
  };

  // a finished tile: scale, then the epilogue (one split) or the FP32 partial (several)
  auto finish = [&](int tile) {
    const int row = tile * 16 + m_row;
    const float rs = rs_s[(tile - tile0) * 16 + m_row];
    if constexpr (MF) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 4 * g + i;
        const float v = acc_m[i] * pscale[t & 15];
        if (a.ks == 1) {
          const float vs = v * rs;
          const float up = __shfl_down(vs, 8, 16);
          if (t < cnt) emit_row(a, epilogue_of(a, expert), pairs ? pairs_s[t] : t, cnt, tile, true, m_row, t, vs, up);
        } else if (t < cnt) {
          a.part[((long long)split * a.m + t) * n_pad + row] = v;
        }
        acc_m[i] = 0.0f;
      }
    } else {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const float v = quad16_sum(acc_v[t]);
        if (a.ks == 1) {
          const float vs = v * rs;
          const float up = __shfl_down(vs, 8, 16);
          if (g == 0 && t < cnt)
            emit_row(a, epilogue_of(a, expert), pairs ? pairs_s[t] : t, cnt, tile, true, m_row, t, vs, up);
        } else if (g == 0 && t < cnt) {
          a.part[((long long)split * a.m + t) * n_pad + row] = v;
        }
        acc_v[t] = 0.0f;
      }
    }
  };

  // ---- the stream: compute unit i, refill its ring slot with unit i + D ----------------------------------------
  int ct = 0, cc = 0;
  if constexpr (PIECES) {
    // steps of 16 units = two scale groups: unit base + i computes with piece i / 8; the piece of the group two
    // ahead is loaded when that group's first unit is issued (i = 0 → slot 1 … no: slot of group (base+i+8)/8)
    for (int base = 0; base < total; base += 16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (base + i < total) {
          compute(ring[i & 7], cc, i >> 3, 0u);
          if (++cc == kw) {
            finish(tile0 + wave + ct * S);
            cc = 0;
            ++ct;
          }
        }
        if ((i & 7) == 0 && base + i + 8 < total) {
          // unit base + i + 8 starts a group (split width a multiple of 8): its piece goes to the slot of its
          // group parity, ((base + i + 8) / 8) & 1 = (i >> 3) ^ 1, free since group (base + i) / 8 - 1 is done
          const uint8_t* tb = wmat + (long long)(tile0 + wave + lt * S) * a.tile_stride;
          spc[(i >> 3) ^ 1] = piece_of(tb, kb + lc);
        }
        load_next(ring[i & 7]);
      }
    }
  } else {
    for (int base = 0; base < total; base += D) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        if (base + i < total) {
          compute(ring[i], cc, 0, ring[i].s);
          if (++cc == kw) {
            finish(tile0 + wave + ct * S);
            cc = 0;
            ++ct;
          }
        }
        load_next(ring[i]);
      }
    }
  }
}

// the K splits of gemv_tk added in split order, scaled by the row scale, through the epilogue
__global__ __launch_bounds__(256) void gemv_tk_reduce(Args a) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const bool silu = a.epilogue == MI_EPI_SILU_MUL || a.epilogue == MI_EPI_SILU_MUL_ROUNDED;
  const int n_out = silu ? a.n / 2 : a.n;
  if (c >= n_out) return;
  const int n_pad = a.n_tiles * 16;
  auto sum = [&](int row) {
    float v = 0.0f;
    for (int s = 0; s < a.ks; ++s) v += a.part[((long long)s * a.m + t) * n_pad + row];
    return v * (a.row_scale != nullptr ? a.row_scale[row] : 1.0f);
  };
  if (silu) {
    const int tile = c / 8, i = c % 8;
    const float gv = sum(tile * 16 + i), uv = sum(tile * 16 + 8 + i);
    float o;
    if (a.epilogue == MI_EPI_SILU_MUL_ROUNDED) o = silu_f(round_bf16(gv)) * round_bf16(uv);
    else o = silu_f(gv) * uv;
    store_out(a, (long long)t * a.ldy + c, o);
  } else {
    float o = sum(c);
    if (a.epilogue == MI_EPI_RESIDUAL) o += bf16_bits_to_f32(a.res[(long long)t * a.ldr + c]);
    store_out(a, (long long)t * a.ldy + c, o);
  }
}

// The split-K reduction of a dense GEMV with BF16 output (epilogue none or residual) and the next RMSNorm of its
// output in one launch: y as gemv_tk_reduce writes it (splits added in order, row scale, residual, one BF16
// rounding), then x_next as norm_apply computes it over y. One workgroup of RN_NT threads per token, a thread per
// 8-column vector: all its loads (partials of every split at a clamped index, residual, row scales, norm weights)
// issued up front, so the launch waits one memory round trip; y goes to LDS, where the first RN_SUM threads take
// Σ y² exactly as norm_apply's threads do (vectors tid, tid + RN_SUM, … in order, fma, then the waves in order) —
// the same statistic, bit for bit — and every thread normalizes its vector (n <= 8·RN_NT, at most RN_KS splits).
constexpr int RN_NT = 1024;
constexpr int RN_SUM = 256;     // norm_apply's workgroup: its per-thread vectors fix the order of Σ
constexpr int RN_KS = 4;
__global__ __launch_bounds__(RN_NT) void gemv_reduce_norm(Args a) {
  __shared__ __attribute__((aligned(16))) uint4 ys[RN_NT];
  __shared__ float red[RN_SUM / 64];
  __shared__ float rsh;
  const int t = blockIdx.x, tid = threadIdx.x;
  const int n_pad = a.n_tiles * 16, nv = a.n / 8;
  const bool resid = a.epilogue == MI_EPI_RESIDUAL;
  const int c = 8 * min(tid, nv - 1);
  float4 pp[RN_KS][2];
#pragma unroll
  for (int sp = 0; sp < RN_KS; ++sp) {
    const float* p = a.part + ((long long)min(sp, a.ks - 1) * a.m + t) * n_pad + c;
    pp[sp][0] = *reinterpret_cast<const float4*>(p);
    pp[sp][1] = *reinterpret_cast<const float4*>(p + 4);
  }
  const float* rsp = a.row_scale != nullptr ? a.row_scale + c : a.nn_w + c;   // the weights stand in: unused
  const float4 rs0 = *reinterpret_cast<const float4*>(rsp), rs1 = *reinterpret_cast<const float4*>(rsp + 4);
  // no residual: a placeholder load from the (read-only) norm weights, whose value goes unused
  const uint4 rq = *reinterpret_cast<const uint4*>(
      (resid ? a.res + (long long)t * a.ldr : reinterpret_cast<const uint16_t*>(a.nn_w)) + c);
  const float4 w0 = *reinterpret_cast<const float4*>(a.nn_w + c), w1 = *reinterpret_cast<const float4*>(a.nn_w + c + 4);
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < RN_KS; ++sp) {
    const bool on = sp < a.ks;
    const float pv[8] = {pp[sp][0].x, pp[sp][0].y, pp[sp][0].z, pp[sp][0].w,
                         pp[sp][1].x, pp[sp][1].y, pp[sp][1].z, pp[sp][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = on ? v[e] + pv[e] : v[e];     // a select: an absent split leaves v as is
  }
  const float rsv[8] = {rs0.x, rs0.y, rs0.z, rs0.w, rs1.x, rs1.y, rs1.z, rs1.w};
  const uint32_t rw[4] = {rq.x, rq.y, rq.z, rq.w};
  uint32_t yb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float lo = v[2 * i] * (a.row_scale != nullptr ? rsv[2 * i] : 1.0f);
    float hi = v[2 * i + 1] * (a.row_scale != nullptr ? rsv[2 * i + 1] : 1.0f);
    if (resid) {
      lo += bf16_bits_to_f32(rw[i] & 0xFFFFu);
      hi += bf16_bits_to_f32(rw[i] >> 16);
    }
    yb[i] = f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
  }
  const uint4 y4{yb[0], yb[1], yb[2], yb[3]};
  if (tid < nv) {
    *reinterpret_cast<uint4*>(a.y + (long long)t * a.ldy + 8 * tid) = y4;
    ys[tid] = y4;
  }
  lds_barrier();
  if (tid < RN_SUM) {
    float s = 0.0f;
    for (int jj = tid; jj < nv; jj += RN_SUM) {
      const uint4 q = ys[jj];
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16_bits_to_f32(qw[i] & 0xFFFFu), hi = bf16_bits_to_f32(qw[i] >> 16);
        s = fmaf(lo, lo, s);
        s = fmaf(hi, hi, s);
      }
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
  }
  lds_barrier();
  if (tid == 0) {
    float ssq = 0.0f;
#pragma unroll
    for (int w = 0; w < RN_SUM / 64; ++w) ssq += red[w];
    rsh = 1.0f / sqrtf(ssq / (float)a.n + a.nn_eps);
  }
  lds_barrier();
  const float r = rsh;
  const float w8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = round_bf16((bf16_bits_to_f32(yb[i] & 0xFFFFu) * r) * w8[2 * i]);
    const float hi = round_bf16((bf16_bits_to_f32(yb[i] >> 16) * r) * w8[2 * i + 1]);
    o[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
  }
  if (tid < nv) *reinterpret_cast<uint4*>(a.nn_x + (long long)t * a.ld_nn_x + 8 * tid) = uint4{o[0], o[1], o[2], o[3]};
}

// ---- exact dequantization through the same decode ---------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(64) void dequant_t16(const uint8_t* w, const float* row_scale, int n, int k, int chunks,
                                                   float* out) {
  const int lane = threadIdx.x;
  const int tile = blockIdx.x / chunks, c = blockIdx.x % chunks;
  Units<FMT> u;
  load_chunk<FMT, true>(u, w + (long long)tile * tile_bytes(FMT, chunks), c, chunks, lane);
  const int row = tile * 16 + (lane & 15), g = lane >> 4;
  if (row >= n) return;
  float* o = out + (long long)row * k;
  const uint32_t dw[4] = {u.q.x, u.q.y, u.q.z, u.q.w};
  if constexpr (FMT == FMT_NVFP4) {
    const ScalePair sp = nvfp4_scales(u.s);
    const float rs = row_scale ? row_scale[row] : 1.0f;
    for (int s = 0; s < 4; ++s) {
      const f16x8 v = nvfp4_decode8(dw[s], s < 2 ? sp.e0 : sp.e1, s < 2 ? sp.m0 : sp.m1);
      for (int i = 0; i < 8; ++i) o[c * 128 + 32 * g + 8 * s + i] = (float)v[i] * rs;
    }
  } else if constexpr (FMT == FMT_INT4) {
    for (int s = 0; s < 4; ++s) {
      const f16x8 v = int4_decode8(dw[s]);
      const uint32_t pr = s < 2 ? u.sb.x : u.sb.y;
      const float sc = bf16_bits_to_f32(pr & 0xFFFFu), bi = bf16_bits_to_f32(pr >> 16);
      for (int i = 0; i < 8; ++i) o[c * 128 + 32 * s + 8 * g + int4_perm8(i)] = fmaf((float)v[i], sc, bi);
    }
  } else if constexpr (FMT == FMT_FP8) {
    const float rs = row_scale ? row_scale[row] : 1.0f;
    for (int s = 0; s < 2; ++s) {
      const f16x8 v = fp8_decode8(dw[2 * s], dw[2 * s + 1]);
      for (int i = 0; i < 8; ++i) o[c * 64 + 16 * g + 8 * s + i] = (float)v[i] * rs;
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
  int kernel = 0;          // 1: gemv_row (gemv_rowp when rt > 1), 2: gemv_tk, 3: gemv_rowm
  int S = 1;               // waves per workgroup
  int kw = 0;              // gemv_row: KW (chunks per wave); gemv_tk: chunks per split
  int tb = 1, ks = 1, depth = 8;   // gemv_tk: tiles per workgroup, K splits, ring depth
  int rt = 1, G = 0;       // gemv_row: tiles per workgroup (at most), workgroups along the tiles
  int lds_rows = 1, row_ld = 0, row_wave_lds = 0;
  size_t lds_bytes = 0;
  bool prenorm = false;    // the input norm as its own norm_apply launch into the workspace, then the plain GEMV
  int passes = 1;          // gemv_row over more than two tokens or pairs: workgroups of two along grid z
};

int check_desc(const mi_gemv_desc* d) {
  MI_REQUIRE(d, "mi_gemv: null descriptor");
  MI_REQUIRE(d->format == FMT_NVFP4 || d->format == FMT_INT4 || d->format == FMT_BF16 || d->format == FMT_FP8,
             "mi_gemv: unknown format %d",
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
  {
    const auto silu = [](int e) { return e == MI_EPI_SILU_MUL || e == MI_EPI_SILU_MUL_ROUNDED; };
    MI_REQUIRE(!d->groups || d->shared_expert <= 0 || (silu(d->shared_epilogue) == silu(d->epilogue) &&
                                                       d->shared_epilogue != MI_EPI_RESIDUAL),
               "mi_gemv: the shared expert's epilogue must give the routed experts' output width (no residual)");
  }
  if (d->route_logits) {
    const int ks = d->route_top_k + (d->shared_expert > 0 ? 1 : 0);
    MI_REQUIRE(d->groups && d->m == 1 && d->route_experts >= 1 && d->route_experts <= 64 * ROUTE_MAX_PER_LANE &&
                   d->route_top_k >= 1 && d->route_top_k <= ROUTE_MAX_K && d->route_top_k <= d->route_experts &&
                   d->top_k == ks && d->max_groups == ks && d->route_ids && d->route_weights &&
                   d->route_ld >= d->route_experts &&
                   (d->shared_expert <= 0 || (d->shared_expert >= d->route_experts &&
                                              d->shared_expert <= 64 * ROUTE_MAX_PER_LANE && d->route_gate_col >= 0 &&
                                              d->route_gate_col < d->route_ld)),
               "mi_gemv: routing in the launch needs one token, groups = slots = route_top_k (+1 with the shared "
               "expert, index <= 512, its gate column inside the route_ld-wide logits row), 1..512 experts, "
               "top_k <= 16 and the route outputs");
  }
  if (d->next_norm_w) {
    MI_REQUIRE(!d->groups && !d->out_f32 && (d->epilogue == MI_EPI_NONE || d->epilogue == MI_EPI_RESIDUAL),
               "mi_gemv: the next norm follows a dense GEMV with a BF16 output (epilogue none or residual)");
    MI_REQUIRE(d->n % 8 == 0 && ((uintptr_t)d->y & 15) == 0 && d->ldy % 8 == 0 && ((uintptr_t)d->next_norm_w & 15) == 0,
               "mi_gemv: the next norm needs n %% 8 == 0, a 16-byte aligned y with ldy %% 8 == 0 and next_norm_w");
    MI_REQUIRE(d->next_x && ((uintptr_t)d->next_x & 15) == 0 && d->ld_next_x >= d->n && d->ld_next_x % 8 == 0,
               "mi_gemv: next_x must be 16-byte aligned rows with ld_next_x >= n, multiple of 8");
  }
  MI_REQUIRE(((uintptr_t)d->x & 15) == 0 && d->ldx % 8 == 0, "mi_gemv: x must be 16-byte aligned with ldx %% 8 == 0");
  MI_REQUIRE(((uintptr_t)d->w & 15) == 0, "mi_gemv: weight pack must be 16-byte aligned");
  MI_REQUIRE(!d->norm_w || ((uintptr_t)d->norm_w & 15) == 0, "mi_gemv: norm_w must be 16-byte aligned");
  if (d->gnorm_w) {
    MI_REQUIRE(!d->norm_w, "mi_gemv: norm_w and gnorm_w are exclusive");
    MI_REQUIRE(d->format == FMT_NVFP4 || d->format == FMT_INT4,
               "mi_gemv: the gated head norm is built for 128-column chunks (NVFP4, INT4)");
    MI_REQUIRE(d->k % 128 == 0, "mi_gemv: gated head norm needs k %% 128 == 0");
    MI_REQUIRE(d->gnorm_z && ((uintptr_t)d->gnorm_z & 15) == 0 && d->ld_gnorm_z % 8 == 0 && d->ld_gnorm_z >= d->k,
               "mi_gemv: gnorm_z must be 16-byte aligned with ld_gnorm_z %% 8 == 0 and >= k");
    MI_REQUIRE(((uintptr_t)d->gnorm_w & 15) == 0, "mi_gemv: gnorm_w must be 16-byte aligned");
  }
  if (d->conv_w) {
    MI_REQUIRE(!d->groups && d->m <= 2 && !d->out_f32 && d->epilogue == MI_EPI_NONE,
               "mi_gemv: the fused conv runs on a dense projection of at most 2 tokens with a plain BF16 output");
    MI_REQUIRE(d->conv_row0 >= 0 && d->conv_row0 % 16 == 0 && d->conv_channels > 0 && d->conv_channels % 16 == 0 &&
                   d->conv_row0 + d->conv_channels <= d->n,
               "mi_gemv: conv rows [%d, %d) must be whole tiles inside the %d outputs", d->conv_row0,
               d->conv_row0 + d->conv_channels, d->n);
    MI_REQUIRE(d->conv_in && d->conv_out && d->ld_conv >= d->conv_channels && ((uintptr_t)d->conv_w & 7) == 0 &&
                   (d->conv_step ? !d->conv_out_state : (d->conv_out_state && d->conv_out_state != d->conv_in)),
               "mi_gemv: the conv needs conv_in, conv_out (ld_conv >= channels), 8-byte aligned taps, and either "
               "conv_step (two slots in conv_in) or a distinct conv_out_state");
  }
  return MI_OK;
}

constexpr size_t kMaxLds = 160 * 1024;

template <int FMT, int MT, int KW> __global__ void gemv_rowp(Args a);

// compute units of the current device (256 on MI355X; also the answer where no device is visible)
int cu_count() {
  static int cached[64] = {0};
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && cached[dev] > 0) return cached[dev];
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
      hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev >= 0 && dev < 64) cached[dev] = n;
  return n;
}

// resident gemv_rowp workgroups per CU for this instantiation, block size and LDS (the occupancy calculator; without
// a device, the wave-slot bound of 32 waves per CU)
int row_blocks_query(int fmt, int kw, int threads, size_t lds) {
  const void* k = nullptr;
#define MI_ROW_K(F, W) if (fmt == F && kw == W) k = reinterpret_cast<const void*>(gemv_rowp<F, 1, W>);
  MI_ROW_K(FMT_NVFP4, 4) MI_ROW_K(FMT_NVFP4, 8) MI_ROW_K(FMT_NVFP4, 16)
  MI_ROW_K(FMT_INT4, 4) MI_ROW_K(FMT_INT4, 8) MI_ROW_K(FMT_INT4, 16)
  MI_ROW_K(FMT_BF16, 4) MI_ROW_K(FMT_BF16, 8) MI_ROW_K(FMT_BF16, 16)
  MI_ROW_K(FMT_FP8, 4) MI_ROW_K(FMT_FP8, 8) MI_ROW_K(FMT_FP8, 16)
#undef MI_ROW_K
  int n = 0;
  if (k && hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, threads, lds) == hipSuccess && n > 0) return n;
  (void)hipGetLastError();
  return std::max(1, 32 / (threads / 64));
}

int row_blocks_per_cu(int fmt, int kw, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, size_t, int>, int> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  (void)hipGetLastError();
  const auto key = std::make_tuple(fmt, kw, threads, lds, dev);
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  const int n = row_blocks_query(fmt, kw, threads, lds);
  std::lock_guard<std::mutex> lk(mu);
  cache[key] = n;
  return n;
}

// gemv_row for M <= 2: KW = 4 while a split's K fits 16 slices of 4 chunks, else 8, else 16 (more, shorter waves keep
// more loads in flight). One K split, except long K over few tiles (N = 5120, K = 17408: 320 workgroups leave a
// quarter of the CUs a second round) where three splits with FP32 partials measured ~10 % faster; a fused norm or
// a grouped (MoE) launch always takes one split.
Plan plan_row(const mi_gemv_desc* d, int fmt, int chunks, int rows, int n_tiles, int groups, int kw_pref = 0) {
  Plan best{};
  double best_cost = 1e30;
  int force_ks = 0, force_kw = kw_pref, force_rt = 0;
  if (const char* env = getenv("MI_GEMV_ROW")) {                                 // tuning sweeps
    const char* ke = getenv("MI_GEMV_ROW_K");                                    // only launches of this K
    if (!ke || atoi(ke) == d->k) sscanf(env, "%d,%d,%d", &force_kw, &force_ks, &force_rt);
  }
  // a long single-split launch without a fused norm takes gemv_rowp too where it needs three or more tiles per
  // resident workgroup (gate|up alone, 2176 tiles: 3–6 % faster in same-box A/B); MI_GEMV_NO_ROWP=1 keeps gemv_row
  static const bool no_rowp = getenv("MI_GEMV_NO_ROWP") && atoi(getenv("MI_GEMV_NO_ROWP")) == 1;
  for (int ks : {1, 3, 2, 4}) {
    if (force_ks && ks != force_ks) continue;
    if (ks > 1 && d->groups) break;
    int kc = (chunks + ks - 1) / ks;
    if (fmt == FMT_NVFP4 && ks > 1) kc = (kc + 7) / 8 * 8;      // splits on scale-group boundaries
    if (ks > 1 && (ks - 1) * kc >= chunks) continue;
    int kw = kc <= 64 ? 4 : kc <= 128 ? 8 : kc <= 160 ? 16 : 0;
    if (force_kw) kw = force_kw;
    if (fmt == FMT_NVFP4 && ks > 1 && kw == 4 && kc % 4) continue;
    if (kw <= 0) continue;
    const int S = (kc + kw - 1) / kw;
    if (S > (kw == 16 ? 10 : 16)) continue;
    const int kcols = chunk_cols(fmt);
    const int ld = kw * kcols + 8;
    size_t wl = (size_t)rows * ld * 2 + (fmt == FMT_INT4 ? (size_t)rows * kw * 8 * 4 : 0);
    wl = (wl + 15) / 16 * 16;
    const size_t lds1 = (size_t)S * wl + (size_t)S * 2 * 4;     // + red[rt][S][rows][16]
    const size_t red1 = (size_t)S * rows * 16 * 4;
    if (lds1 + red1 > kMaxLds) continue;
    // gemv_rowp (rt > 1 tiles per workgroup) where the input norm is fused: its statistic then costs once per
    // workgroup instead of once per tile; rt is what keeps ~every workgroup resident at once
    int rt = 1;
    if (rows == 1 && !d->groups && (d->norm_w || force_rt || (ks == 1 && !no_rowp))) {
      const int per_cu = row_blocks_per_cu(fmt, kw, 64 * S, lds1 + 4 * red1);
      const long long slots = (long long)cu_count() * std::max(per_cu, 1);
      rt = (int)std::min<long long>(4, std::max<long long>(1, ((long long)n_tiles * ks + slots - 1) / slots));
      if (rt < 3) rt = 1;          // measured: at two tiles per workgroup the loop costs what the statistic saves
      if (force_rt) rt = force_rt;
    }
    const size_t lds = lds1 + (size_t)rt * red1;
    const int want_ks = (chunks >= 96 && n_tiles * groups <= 512 && !d->norm_w && !d->groups) ? 3 : 1;
    const double cost = force_ks ? 0.0 : std::abs(ks - want_ks);
    if (cost < best_cost) {
      best_cost = cost;
      best = Plan{};
      best.kernel = 1; best.S = S; best.kw = kw; best.ks = ks; best.tb = kc; best.lds_rows = rows; best.row_ld = ld;
      best.row_wave_lds = (int)wl; best.lds_bytes = lds;
      best.rt = rt; best.G = n_tiles;
      if (rt > 1) {                            // every resident slot takes tiles (strided): no idle CUs
        best.G = force_rt ? (n_tiles + rt - 1) / rt : (int)std::min<long long>(n_tiles, (long long)cu_count() *
                 std::max(row_blocks_per_cu(fmt, kw, 64 * S, lds1 + 4 * red1), 1));
        best.rt = (n_tiles + best.G - 1) / best.G;
        best.lds_bytes = lds1 + (size_t)best.rt * red1;
      }
    }
  }
  return best;
}

int tk_lds(int fmt, int rows, int kc, bool mf) {
  const int kcols = chunk_cols(fmt);
  size_t b = (size_t)rows * (kc * kcols + 8) * 2 + 16 * 4;
  if (fmt == FMT_INT4) b += mf ? (size_t)kc * 2 * 16 * 4 : (size_t)rows * kc * 8 * 4;
  b += 64;
  return (int)((b + 15) / 16 * 16);
}

// gemv_tk: K splits (ks), tiles per workgroup (tb), waves per workgroup (S), ring depth (D ∈ {4, 8, 12}), chosen by
// a bytes-over-rate model: the rate falls off below ~96 KB of weights in flight per CU; the activations cost their
// re-reads (workgroups × split bytes), split K its partials and a second launch; a fused norm needs one split.
Plan plan_tk(const mi_gemv_desc* d, int fmt, int chunks, int n_tiles, int groups, int rows) {
  Plan best{};
  if (fmt == FMT_FP8) return best;            // no FP8 path in gemv_tk
  const bool mf = rows > 2;
  int force[4] = {0, 0, 0, 0};           // MI_GEMV_TK="ks,tb,S,D" pins a plan (tuning sweeps)
  if (const char* env = getenv("MI_GEMV_TK")) sscanf(env, "%d,%d,%d,%d", &force[0], &force[1], &force[2], &force[3]);
  const int ub = unit_bytes(fmt);
  double best_cost = 1e30;
  for (int ks = 1; ks <= 16; ++ks) {
    if (force[0] && ks != force[0]) continue;
    if (ks > 1 && d->groups) break;
    int kc = (chunks + ks - 1) / ks;
    if (fmt == FMT_NVFP4 && ks > 1) kc = (kc + 7) / 8 * 8;   // splits on scale-group boundaries
    if (ks > 1 && (ks - 1) * kc >= chunks) continue;    // no empty split
    const int lrows = mf ? std::min(16, rows) : rows;
    const int lds = tk_lds(fmt, lrows, kc, mf);
    if (lds > 96 * 1024) continue;
    for (int S : {1, 2, 4, 8}) {
      if (force[2] && S != force[2]) continue;
      for (int tb = S; tb <= 8 * S; tb += S) {
        if (force[1] && tb != force[1]) continue;
        if (tb > n_tiles && tb != S) break;
        for (int D : {4, 8, 12}) {
          if (force[3] && D != force[3]) continue;
          // NVFP4 on whole scale groups streams with D = 8 (the piece ring); otherwise any depth
          if (fmt == FMT_NVFP4 && chunks % 8 == 0 && kc % 8 == 0 && D != 8) continue;
          // INT4 on the matrix path: a deeper ring costs more in occupancy than it adds in flight (27B gate|up at
          // M = 8: D = 4 32.5 µs, D = 8 35.0 µs, the D = 12 plan the model preferred 52.7 µs)
          if (fmt == FMT_INT4 && mf && D != 4) continue;
          const int lds_t = lds + tb * 16 * 4 + 64;   // + the staged row scales and pair ids
          const double wgs = (double)((n_tiles + tb - 1) / tb) * ks * groups;
          const int per_cu_lds = std::max(1, (int)(kMaxLds / lds_t));
          const int per_cu = std::min(per_cu_lds, 32 / S);
          const double resident_waves = std::min(wgs, 256.0 * per_cu) * S / 256.0;
          const double inflight = resident_waves * D * ub;
          const double rounds = wgs / (256.0 * per_cu);
          const double tail = rounds > 1.0 ? std::ceil(rounds) / rounds : 1.0;
          const double w_bytes = (double)n_tiles * chunks * ub * groups;
          const double x_bytes = wgs * lrows * kc * chunk_cols(fmt) * 2.0;
          const double p_bytes = ks > 1 ? 2.0 * ks * rows * n_tiles * 16 * 4 : 0.0;
          const double rate = std::min(1.0, inflight / (96.0 * 1024));
          double cost = (w_bytes + 0.5 * x_bytes + p_bytes) / std::max(rate, 1e-3) * tail;
          cost += ks > 1 ? w_bytes * 0.12 : 0.0;
          const int lw = ((n_tiles + tb - 1) / tb) * tb - n_tiles;
          cost *= 1.0 + (double)lw / n_tiles;
          if (cost < best_cost) {
            best_cost = cost;
            best.kernel = 2; best.S = S; best.kw = kc; best.tb = tb; best.ks = ks; best.depth = D;
            best.lds_rows = lrows; best.lds_bytes = lds_t;
          }
        }
      }
    }
  }
  // A weight stream larger than the MALL (the BF16 lm_head, 2.54 GB at M = 8): at most two tiles per wave, so four
  // times the workgroups stream at once — measured 383–403 µs against 412–420 µs for the model's 64 tiles (the
  // model's in-flight estimate already saturates there)
  if (best.kernel == 2 && !force[1] && (double)n_tiles * chunks * ub * groups > 256.0 * (1 << 20) && best.tb > 2 * best.S)
    best.tb = 2 * best.S;
  return best;
}

// gemv_rowm (3 <= M <= 16, NVFP4 / FP8 / INT4): waves of 512 columns over K splits of at most 12 waves; as many
// workgroups as are resident at once, each over rt tiles
template <int FMT> __global__ void gemv_rowm(Args a);
int rowm_blocks_per_cu(int fmt, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, size_t, int>, int> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  (void)hipGetLastError();
  const auto key = std::make_tuple(threads * 8 + fmt, lds, dev);
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int n = 0;
  const void* kern = fmt == FMT_FP8    ? reinterpret_cast<const void*>(gemv_rowm<FMT_FP8>)
                     : fmt == FMT_INT4 ? reinterpret_cast<const void*>(gemv_rowm<FMT_INT4>)
                                       : reinterpret_cast<const void*>(gemv_rowm<FMT_NVFP4>);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) !=
          hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = std::max(1, 12 / (threads / 64));      // no device: the 3 waves per SIMD of the kernel's VGPR budget
  }
  std::lock_guard<std::mutex> lk(mu);
  cache[key] = n;
  return n;
}

Plan plan_rowm(const mi_gemv_desc* d, int chunks, int n_tiles) {
  Plan best{};
  if ((d->format != FMT_NVFP4 && d->format != FMT_FP8 && d->format != FMT_INT4) || d->groups || d->gnorm_w ||
      d->m < 3 || d->m > 16 ||
      (d->format == FMT_NVFP4 && chunks % 4))     // NVFP4 slices start on half scale groups
    return best;
  const int kw = 512 / chunk_cols(d->format);    // chunks per wave (512 columns)
  int ks = (chunks + 12 * kw - 1) / (12 * kw);   // at most 12 waves: the kernel's VGPR budget is 3 waves per SIMD
  if (d->norm_w && ks > 1) return best;          // the fused norm needs the whole row in one workgroup
  int force_ks = 0, force_rt = 0;
  if (const char* env = getenv("MI_GEMV_ROWM")) {                                // tuning sweeps
    const char* ke = getenv("MI_GEMV_ROWM_K");                                   // only launches of this K
    if (!ke || atoi(ke) == d->k) sscanf(env, "%d,%d", &force_ks, &force_rt);
  }
  if (force_ks) ks = force_ks;
  // one split whose tiles' waves fill under three quarters of the chip's wave slots (12 per CU at this kernel's
  // VGPR budget): three K splits, so the tiles spread over every CU (27B attention o_proj at M = 8, 320 tiles of 6
  // waves: 14.0 → 11.6 µs with the reduction launch; out_proj's 12 waves per tile measured best unsplit)
  if (!force_ks && ks == 1 && !d->norm_w && (long long)n_tiles * ((chunks + kw - 1) / kw) * 4 < 3LL * cu_count() * 12) {
    const int kc3 = ((chunks + 2) / 3 + 7) / 8 * 8;
    if (2 * kc3 < chunks) ks = 3;                // three non-empty splits on scale-group boundaries
  }
  int kc = (chunks + ks - 1) / ks;
  if (ks > 1) kc = (kc + 7) / 8 * 8;             // splits on scale-group boundaries (whole waves for FP8)
  if (kc > 12 * kw || (ks > 1 && (ks - 1) * kc >= chunks)) return best;
  const int S = (kc + kw - 1) / kw;
  const size_t fixed = (d->norm_w ? (size_t)d->k * 4 : 0) + (size_t)S * 16 * 4 +
                       (d->format == FMT_INT4 ? (size_t)S * (512 / chunk_cols(FMT_INT4)) * 2 * 16 * 4 : 0);
  const size_t per_tile = (size_t)S * 16 * 16 * 4;
  const int per_cu = rowm_blocks_per_cu(d->format, 64 * S, fixed + 4 * per_tile);
  const long long slots = std::max<long long>(1, (long long)cu_count() * std::max(per_cu, 1) / ks);
  // every resident slot takes tiles (strided), so no CU idles for the rounding of tiles per workgroup
  int G = (int)std::min<long long>(n_tiles, slots);
  if (force_rt) G = (n_tiles + force_rt - 1) / force_rt;
  const int rt = (n_tiles + G - 1) / G;
  const size_t lds = fixed + (size_t)rt * per_tile;
  if (lds > kMaxLds) return best;
  best.kernel = 3; best.S = S; best.kw = kc; best.ks = ks; best.rt = rt; best.G = G;
  best.tb = rt; best.lds_rows = 16; best.lds_bytes = lds;
  return best;
}

Plan make_plan_fused(const mi_gemv_desc* d);

// split-K workspace: a fixed region of per-tile arrival counters (the same for every shape, so partials of one call
// never land on the counters of another), then the FP32 partials [ks][m][n_tiles·16], then (prenorm) the
// normalized input rows [m][k] BF16
constexpr int kFoldTiles = 16384;
constexpr size_t kFoldCounterBytes = kFoldTiles * sizeof(uint32_t);
size_t fold_counter_bytes(int) { return kFoldCounterBytes; }

// At M >= 3 the input RMSNorm runs as its own norm_apply launch (one workgroup per token) into the workspace, and the
// GEMV reads the normalized rows: inside gemv_rowm / gemv_tk every workgroup would normalize the whole [M, K] input
// again (per element: two multiplies and a BF16 rounding, on operand lanes of which half are padding rows at M = 8)
// behind a workgroup barrier. Measured on the 27B shapes at M = 8, bit-identical: gate|up 33.0 → 30.5 µs, in_proj
// 24.7 → 22.0 µs (the extra launch ≈ 2.9 µs). At M <= 2 gemv_row's fused norm costs less than a launch.
bool wants_prenorm(const mi_gemv_desc* d) {
  static const bool off = getenv("MI_GEMV_PRENORM") && getenv("MI_GEMV_PRENORM")[0] == '0';   // A/B comparisons
  const int rows = d->groups ? std::min(16, d->m) : d->m;
  return !off && d->norm_w && rows > 2 && !(d->groups && d->x_per_slot) && !d->route_logits && d->k % 8 == 0;
}

Plan make_plan(const mi_gemv_desc* d) {
  if (d->conv_w) {                              // the conv epilogue lives in gemv_row: one tile per workgroup
    Plan p = make_plan_fused(d);
    if (p.kernel == 1 && p.rt > 1) {
      p.rt = 1;
      p.G = (d->n + 15) / 16;
      p.lds_bytes = (size_t)p.S * p.row_wave_lds + (size_t)p.S * 2 * 4 + (size_t)p.S * p.lds_rows * 16 * 4;
    }
    return p.kernel == 1 ? p : Plan{};
  }
  if (!wants_prenorm(d)) return make_plan_fused(d);
  mi_gemv_desc plain = *d;
  plain.norm_w = nullptr;
  Plan p = make_plan_fused(&plain);
  p.prenorm = p.kernel != 0;
  return p;
}

// the normalized rows' place in the workspace (after the split-K counters and partials), and the bytes in all
size_t split_bytes(const mi_gemv_desc* d, const Plan& p) {
  return p.ks > 1 ? fold_counter_bytes(d->n) + (size_t)p.ks * d->m * ((d->n + 15) / 16) * 16 * sizeof(float) : 0;
}
// (past the counters also without a split: a workspace is shared between calls, and the counters must stay zero)
size_t prenorm_offset(const mi_gemv_desc* d, const Plan& p) {
  return (std::max(split_bytes(d, p), fold_counter_bytes(d->n)) + 255) / 256 * 256;
}
size_t workspace_need(const mi_gemv_desc* d, const Plan& p) {
  return p.prenorm ? prenorm_offset(d, p) + (size_t)d->m * d->k * sizeof(uint16_t) : split_bytes(d, p);
}

Plan make_plan_fused(const mi_gemv_desc* d) {
  const int fmt = d->format;
  const int chunks = d->k / chunk_cols(fmt);
  const int n_tiles = (d->n + 15) / 16;
  const int groups = d->groups ? d->max_groups : 1;
  const int rows = d->groups ? std::min(16, d->m) : d->m;   // a group holds at most one pair per token
  const char* fk = getenv("MI_GEMV_KERNEL");                 // "row" / "tk" / "rowm" pins the kernel (sweeps)
  const bool pin_tk = fk && fk[0] == 't', pin_rowm = fk && strcmp(fk, "rowm") == 0;
  if (rows <= 2 && !pin_tk) {
    const Plan p = plan_row(d, fmt, chunks, rows, n_tiles, groups);
    // A fused-norm tile per workgroup whose 4-chunk waves leave a second, partial round of workgroups (too few
    // tiles per slot for gemv_rowp): 8 chunks per wave halves the waves per tile, so every tile is resident in one
    // round. 27B in_proj (1030 tiles): 14.7–15.2 → 14.2–14.4 µs; gate|up (gemv_rowp) and the shapes without the
    // norm measured best as planned.
    if (p.kernel == 1 && p.rt == 1 && p.ks == 1 && p.kw == 4 && rows == 1 && d->norm_w && !d->groups &&
        fmt == FMT_NVFP4 && chunks % 8 == 0 && !getenv("MI_GEMV_ROW")) {
      const long long slots = (long long)cu_count() * std::max(row_blocks_per_cu(fmt, 4, 64 * p.S, p.lds_bytes), 1);
      if (n_tiles > slots) {
        const Plan p8 = plan_row(d, fmt, chunks, rows, n_tiles, groups, 8);
        if (p8.kernel) return p8;
      }
    }
    // Fewer tiles than half the CUs (the MoE router, 17 BF16 tiles): 8 chunks per wave, half the waves per
    // workgroup — 3.9–4.1 → 3.4–3.5 µs; the grouped expert launches (576 workgroups) are faster with 4
    if (p.kernel == 1 && p.rt == 1 && p.ks == 1 && p.kw == 4 && !getenv("MI_GEMV_ROW") &&
        (long long)n_tiles * groups * 2 < cu_count() && (fmt != FMT_NVFP4 || chunks % 8 == 0)) {
      const Plan p8 = plan_row(d, fmt, chunks, rows, n_tiles, groups, 8);
      if (p8.kernel && p8.ks == 1) return p8;
    }
    if (p.kernel) return p;
  }
  // Grouped (MoE) NVFP4 launches at M >= 3: routing spreads the tokens over the experts, so a group holds one or
  // two pairs (the shared expert's group all of them): gemv_row takes them two per workgroup (grid z: the passes)
  // instead of gemv_tk padding every group to 16 MFMA rows. A small BF16 matrix (the MoE router, 1 MB) the same
  // way, two tokens per workgroup: its passes re-read it from the caches, and no split-K reduction launch follows.
  // (NVFP4 stays on gemv_rowm: the attention o_proj, 8.8 MB, measured 11.8 → 10.5–10.8 µs alone but no faster in
  // the layer; out_proj, 17.7 MB, and q|k|v, 20 MB, are slower with passes)
  const bool small = !d->groups && !d->gnorm_w && fmt == FMT_BF16 && (size_t)d->n * d->k * 2 <= (8u << 20);
  if (rows > 2 && ((d->groups && fmt == FMT_NVFP4) || small) && !pin_tk && !pin_rowm &&
      !(getenv("MI_GEMV_PASSES") && getenv("MI_GEMV_PASSES")[0] == '0')) {       // =0: the earlier plans (A/B)
    Plan p = plan_row(d, fmt, chunks, 2, n_tiles, groups);
    if (p.kernel && p.ks == 1 && p.rt == 1) {
      // records of at most two pairs (mi_moe_route's pairs_per_record): one pass; else the passes along z
      p.passes = d->groups && d->group_max_pairs > 0 && d->group_max_pairs <= 2 ? 1 : (rows + 1) / 2;
      return p;
    }
  }
  // INT4 at M >= 3 runs on gemv_tk unless gemv_rowm is pinned: measured on the 27B gate|up shape at M = 8,
  // gemv_rowm takes 37.4 µs against gemv_tk's 35.5 (its per-group scale / bias work is VALU time the NVFP4 decode
  // does not have), although gemv_tk moves 11 MB of split partials more
  if (rows > 2 && !pin_tk && (fmt != FMT_INT4 || pin_rowm)) {
    const Plan p = plan_rowm(d, chunks, n_tiles);
    if (p.kernel) return p;
  }
  return plan_tk(d, fmt, chunks, n_tiles, groups, rows);
}

// dynamic LDS above 64 KB must be allowed per kernel once
template <typename K>
void allow_lds(K kernel) {
  static std::once_flag once;
  std::call_once(once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kMaxLds);
    (void)hipGetLastError();
  });
}

template <int FMT, int MT>
void launch_tk_d(const Args& a, const Plan& p, dim3 g, hipStream_t s) {
  const bool pieces = FMT == FMT_NVFP4 && a.chunks % 8 == 0 && p.kw % 8 == 0;
  if (pieces) { allow_lds(gemv_tk<FMT, MT, 8, true>); hipLaunchKernelGGL((gemv_tk<FMT, MT, 8, true>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
  else if (p.depth == 4) { allow_lds(gemv_tk<FMT, MT, 4, false>); hipLaunchKernelGGL((gemv_tk<FMT, MT, 4, false>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
  else if (p.depth == 8) { allow_lds(gemv_tk<FMT, MT, 8, false>); hipLaunchKernelGGL((gemv_tk<FMT, MT, 8, false>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
  else { allow_lds(gemv_tk<FMT, MT, 12, false>); hipLaunchKernelGGL((gemv_tk<FMT, MT, 12, false>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
}

template <int FMT, int MT, int KW>
void launch_row_kw(const Args& a, const Plan& p, dim3 g, hipStream_t s) {
  if (MT == 1 && p.rt > 1) { allow_lds(gemv_rowp<FMT, 1, KW>); hipLaunchKernelGGL((gemv_rowp<FMT, 1, KW>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
  else if (a.conv_w) {
    if constexpr (MT <= 2) { allow_lds(gemv_row<FMT, MT, KW, true>); hipLaunchKernelGGL((gemv_row<FMT, MT, KW, true>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
  } else { allow_lds(gemv_row<FMT, MT, KW, false>); hipLaunchKernelGGL((gemv_row<FMT, MT, KW, false>), g, dim3(64 * p.S), p.lds_bytes, s, a); }
}

template <int FMT, int MT>
void launch_row_k(const Args& a, const Plan& p, dim3 g, hipStream_t s) {
  if (p.kw == 4) launch_row_kw<FMT, MT, 4>(a, p, g, s);
  else if (p.kw == 8) launch_row_kw<FMT, MT, 8>(a, p, g, s);
  else launch_row_kw<FMT, MT, 16>(a, p, g, s);
}

// the split-K reduction launch: with the next norm (a.nn_w), gemv_reduce_norm; else gemv_tk_reduce
void launch_reduce(const Args& a, hipStream_t s) {
  if (a.nn_w) {
    hipLaunchKernelGGL(gemv_reduce_norm, dim3(a.m), dim3(RN_NT), 0, s, a);
    return;
  }
  const bool silu = a.epilogue == MI_EPI_SILU_MUL || a.epilogue == MI_EPI_SILU_MUL_ROUNDED;
  const int n_out = silu ? a.n / 2 : a.n;
  hipLaunchKernelGGL(gemv_tk_reduce, dim3((n_out + 255) / 256, a.m), dim3(256), 0, s, a);
}

template <int FMT>
void launch(const Args& a, const Plan& p, int groups, hipStream_t s) {
  if constexpr (FMT == FMT_NVFP4 || FMT == FMT_FP8 || FMT == FMT_INT4) {
    if (p.kernel == 3) {
      allow_lds(gemv_rowm<FMT>);
      hipLaunchKernelGGL(gemv_rowm<FMT>, dim3(p.G, 1, p.ks), dim3(64 * p.S), p.lds_bytes, s, a);
      if (p.ks > 1) launch_reduce(a, s);
      return;
    }
  }
  if (p.kernel == 1) {
    const dim3 g(p.G, groups, p.passes > 1 ? p.passes : p.ks);
    if (p.lds_rows == 2) launch_row_k<FMT, 2>(a, p, g, s);
    else launch_row_k<FMT, 1>(a, p, g, s);
    if (p.ks > 1 && !a.fold_cnt) launch_reduce(a, s);
    return;
  }
  if constexpr (FMT != FMT_FP8) {                // FP8 runs on gemv_row / gemv_rowm only (the planner's choice)
    const dim3 g((a.n_tiles + p.tb - 1) / p.tb, p.ks, groups);
    if (p.lds_rows > 2) launch_tk_d<FMT, 16>(a, p, g, s);
    else if (p.lds_rows == 2) launch_tk_d<FMT, 2>(a, p, g, s);
    else launch_tk_d<FMT, 1>(a, p, g, s);
    if (p.ks > 1) launch_reduce(a, s);
  }
}

}  // namespace

extern "C" {

size_t mi_pack_bytes(int32_t format, int32_t n, int32_t k) {
  if (n <= 0 || k <= 0) return 0;
  if (format != FMT_NVFP4 && format != FMT_INT4 && format != FMT_BF16 && format != FMT_FP8) return 0;
  const int kc = chunk_cols(format);
  if (k % kc) return 0;
  return (size_t)((n + 15) / 16) * (size_t)tile_bytes(format, k / kc);
}

size_t mi_gemv_workspace_bytes(const mi_gemv_desc* d) {
  if (check_desc(d) != MI_OK) return 0;
  return workspace_need(d, make_plan(d));
}

int mi_gemv_plan(const mi_gemv_desc* d, int32_t out[7]) {
  if (int rc = check_desc(d)) return rc;
  MI_REQUIRE(out, "mi_gemv_plan: null output");
  const Plan p = make_plan(d);
  MI_REQUIRE(p.kernel, "mi_gemv_plan: no launch plan fits (k=%d, m=%d)", d->k, d->m);
  const int n_tiles = (d->n + 15) / 16;
  const int groups = d->groups ? d->max_groups : 1;
  out[0] = p.kernel; out[1] = p.S; out[2] = p.kw;
  out[3] = p.kernel == 1 ? p.rt : p.tb; out[4] = p.ks; out[5] = (int32_t)p.lds_bytes;
  out[6] = (p.kernel != 2 ? p.G * (p.passes > 1 ? p.passes : p.ks) : (n_tiles + p.tb - 1) / p.tb * p.ks) * groups;
  return MI_OK;
}

}  // extern "C"

namespace {

// The body of mi_gemv and mi_gemv_noalloc. fixed_ws: the split-K buffer to use (the no-allocation entry point's
// device-resident array), or null: the caller's workspace, else the library's scratch.
int gemv_impl(const mi_gemv_desc* d, void* stream, void* fixed_ws, size_t fixed_bytes, const char* name) {
  if (int rc = check_desc(d)) return rc;
  const Plan p = make_plan(d);
  MI_REQUIRE(p.kernel, "%s: no launch plan fits (k=%d, m=%d)", name, d->k, d->m);
  MI_REQUIRE(!d->route_logits || (p.kernel == 1 && p.ks == 1), "%s: routing in the launch runs on gemv_row", name);
  Args a{};
  a.w = static_cast<const uint8_t*>(d->w);
  a.row_scale = d->row_scale;
  a.x = d->x;
  a.y = d->y;
  a.res = d->residual;
  a.norm_w = d->norm_w;
  a.gnorm_w = d->gnorm_w;
  a.gnorm_z = d->gnorm_z;
  a.ld_gnorm_z = d->ld_gnorm_z;
  a.gnorm_eps = d->gnorm_eps;
  a.groups = d->groups;
  a.eps = d->eps;
  a.ldx = d->ldx; a.ldy = d->ldy; a.ldr = d->ldr;
  a.n = d->n; a.k = d->k; a.m = d->m;
  a.n_tiles = (d->n + 15) / 16;
  a.chunks = d->k / chunk_cols(d->format);
  a.tile_stride = tile_bytes(d->format, a.chunks);
  a.expert_stride = (long long)a.n_tiles * a.tile_stride;
  a.epilogue = d->epilogue;
  a.shared_expert = d->groups ? d->shared_expert : 0;
  a.shared_epilogue = d->shared_epilogue;
  a.route_logits = d->route_logits;
  a.route_e = d->route_experts;
  a.route_k = d->route_top_k;
  a.route_renorm = d->route_renorm;
  a.route_gate_col = d->route_gate_col;
  a.route_n = d->max_groups;
  a.route_ids = d->route_ids;
  a.route_weights = d->route_weights;
  a.route_groups = const_cast<int32_t*>(d->groups);
  a.top_k = d->top_k;
  a.x_per_slot = d->x_per_slot;
  a.out_f32 = d->out_f32;
  a.lds_rows = p.lds_rows;
  a.tb = p.tb;
  a.ks = p.ks;
  a.kc = p.kernel == 1 ? p.tb : p.kw;     // chunks per K split
  a.row_ld = p.row_ld;
  a.row_wave_lds = p.row_wave_lds;
  a.passes = d->groups ? 0 : p.passes;
  a.conv_w = d->conv_w;
  a.conv_in = d->conv_in;
  a.conv_out_state = d->conv_out_state;
  a.conv_out = d->conv_out;
  a.conv_row0 = d->conv_row0;
  a.conv_ch = d->conv_channels;
  a.ld_conv = d->ld_conv;
  a.conv_step = d->conv_step;
  a.conv_done = d->conv_done;
  const size_t need = workspace_need(d, p);
  void* ws = nullptr;
  if (need) {
    ws = fixed_ws ? fixed_ws : d->workspace;
    if (fixed_ws) {
      MI_REQUIRE(need <= fixed_bytes, "%s: this shape needs %zu B of scratch, more than the %zu B the "
                 "no-allocation entry point holds (use mi_gemv with a workspace)", name, need, fixed_bytes);
    } else if (ws) {
      MI_REQUIRE(d->workspace_bytes >= need, "%s: workspace %zu B < %zu B", name, d->workspace_bytes, need);
    } else if (int rc = mi_library_scratch(MI_SCRATCH_GEMV, need, static_cast<hipStream_t>(stream), &ws)) {
      return rc;
    }
  }
  if (p.prenorm) {                              // x → bf16(RMSNorm(x)·w) rows in the workspace; the GEMV reads them
    uint16_t* xn = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + prenorm_offset(d, p));
    mi_norm_desc nd{};
    nd.t = d->m; nd.k = d->k; nd.h = d->x; nd.ldh = d->ldx; nd.stat = nullptr; nd.stat_parts = 1;
    nd.w = d->norm_w; nd.x = xn; nd.ldx = d->k; nd.eps = d->eps;
    if (int rc = mi_norm_apply(&nd, stream)) return rc;
    a.x = xn;
    a.ldx = d->k;
    a.norm_w = nullptr;
  }
  if (p.ks > 1) {
    const size_t cb = fold_counter_bytes(d->n);
    a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + cb);
    // gemv_row folds its splits in the kernel (MI_GEMV_FOLD=0: the separate reduction launch, for comparisons)
    static const bool fold = !(getenv("MI_GEMV_FOLD") && getenv("MI_GEMV_FOLD")[0] == '0');
    if (p.kernel == 1 && fold && a.n_tiles <= kFoldTiles) a.fold_cnt = static_cast<uint32_t*>(ws);
  }
  MI_REQUIRE(!d->conv_w || p.ks == 1 || a.fold_cnt, "%s: the fused conv needs the K splits folded in the kernel", name);
  // the next RMSNorm of y: computed by the split-K reduction launch where the plan has one and the row fits one
  // workgroup's registers; otherwise a norm_apply launch after the GEMV (the same values either way)
  const bool reduce_launch = p.ks > 1 && !a.fold_cnt && p.passes <= 1;
  const bool nn_fused = d->next_norm_w && reduce_launch && d->n <= 8 * RN_NT && p.ks <= RN_KS &&
                        (d->epilogue != MI_EPI_RESIDUAL || (((uintptr_t)d->residual & 15) == 0 && d->ldr % 8 == 0));
  if (nn_fused) {
    a.nn_w = d->next_norm_w;
    a.nn_x = d->next_x;
    a.ld_nn_x = d->ld_next_x;
    a.nn_eps = d->next_eps;
  }
  const int groups = d->groups ? d->max_groups : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->format == FMT_NVFP4) launch<FMT_NVFP4>(a, p, groups, s);
  else if (d->format == FMT_INT4) launch<FMT_INT4>(a, p, groups, s);
  else if (d->format == FMT_FP8) launch<FMT_FP8>(a, p, groups, s);
  else launch<FMT_BF16>(a, p, groups, s);
  MI_TRY_HIP(hipGetLastError(), "gemv launch");
  if (d->next_norm_w && !nn_fused) {
    mi_norm_desc nd{};
    nd.t = d->m; nd.k = d->n; nd.h = d->y; nd.ldh = d->ldy; nd.stat = nullptr; nd.stat_parts = 1;
    nd.w = d->next_norm_w; nd.x = d->next_x; nd.ldx = d->ld_next_x; nd.eps = d->next_eps;
    if (int rc = mi_norm_apply(&nd, stream)) return rc;
  }
  return MI_OK;
}

// ---- the no-allocation entry point's scratch: one device-resident array per GPU, found once per device with
// hipGetSymbolAddress (the array's host-side name is not a device address) ------------------------------------------
constexpr size_t kNoAllocScratchBytes = 8u << 20;   // fold counters (64 KiB) + split-K partials
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

__global__ void clear_words(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

std::mutex g_noalloc_mu;
std::vector<void*> g_noalloc_ptr;     // per device: the address of that device's copy of `scratch`, or null

// the current device's scratch address; on a device's first call its fold counters are cleared by a small fill
// kernel on the caller's stream (ordered before this call's kernels; captured with them if the caller captures)
int noalloc_scratch(hipStream_t s, void** out) {
  int dev = 0;
  MI_TRY_HIP(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if ((int)g_noalloc_ptr.size() <= dev) g_noalloc_ptr.resize(dev + 1, nullptr);
  if (!g_noalloc_ptr[dev]) {
    void* ptr = nullptr;
    MI_TRY_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    hipLaunchKernelGGL(clear_words, dim3(16), dim3(256), 0, s, static_cast<uint32_t*>(ptr),
                       (int)(kFoldCounterBytes / sizeof(uint32_t)));
    MI_TRY_HIP(hipGetLastError(), "clear_words launch");
    g_noalloc_ptr[dev] = ptr;
  }
  *out = g_noalloc_ptr[dev];
  return MI_OK;
}

}  // namespace

extern "C" {

int mi_gemv(const mi_gemv_desc* d, void* stream) { return gemv_impl(d, stream, nullptr, 0, "mi_gemv"); }

int mi_gemv_noalloc(const mi_gemv_desc* d, void* stream) {
  MI_REQUIRE(d, "mi_gemv_noalloc: null descriptor");
  MI_REQUIRE(!d->workspace, "mi_gemv_noalloc: takes no workspace (its split-K scratch is the library's fixed "
             "device array); pass workspace = NULL");
  void* ws = nullptr;
  if (int rc = noalloc_scratch(static_cast<hipStream_t>(stream), &ws)) return rc;
  return gemv_impl(d, stream, ws, kNoAllocScratchBytes, "mi_gemv_noalloc");
}

size_t mi_gemv_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int mi_dequant(int32_t format, const void* w, const float* row_scale, int32_t n, int32_t k, float* out, void* stream) {
  MI_REQUIRE(w && out, "mi_dequant: null pointer");
  MI_REQUIRE(format == FMT_NVFP4 || format == FMT_INT4 || format == FMT_BF16 || format == FMT_FP8,
             "mi_dequant: unknown format");
  const int kc = chunk_cols(format);
  MI_REQUIRE(n > 0 && k > 0 && k % kc == 0, "mi_dequant: bad shape");
  const int chunks = k / kc, tiles = (n + 15) / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  if (format == FMT_NVFP4)
    hipLaunchKernelGGL(dequant_t16<FMT_NVFP4>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  else if (format == FMT_INT4)
    hipLaunchKernelGGL(dequant_t16<FMT_INT4>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  else if (format == FMT_FP8)
    hipLaunchKernelGGL(dequant_t16<FMT_FP8>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  else
    hipLaunchKernelGGL(dequant_t16<FMT_BF16>, dim3(tiles * chunks), dim3(64), 0, s, wb, row_scale, n, k, chunks, out);
  MI_TRY_HIP(hipGetLastError(), "dequant_t16 launch");
  return MI_OK;
}

}  // extern "C"
