// GQA decode attention over an int8 or BF16 KV cache, T new tokens (ops/attention.py `gqa_decode` + `gqa_merge`;
// nn/attention.py:215-243; nn/oracle.py:112-134; kernels/common/gqa_decode.metal:32-302).
//
// Semantics: q|gate per head, k, v from the projection; optional q/k RMSNorm(1 + w); partial RoPE (rotate_half on
// the first rotary_dim dims, BF16 arithmetic, BF16 tables); the fresh k/v are quantized into the cache
// (per token and KV head: scale = f16(absmax / 127), code = rint(x / scale)); scores bf16(bf16(q·k)·D^-½) over the
// dequantized cache, causal inside the step; softmax in FP32 with P rounded to BF16; P·V in FP32 → BF16;
// × bf16(σ(gate)). With the BF16 cache (the reference's own, nn/attention.py:87-89) the fresh k/v are stored as they
// are and the scores use them directly. Head dims 128 and 256 (the reference's 27B attention layer is 24/4/256).
//
// MI355X design, one launch (two where the partials are many):
//  * Cache layout (this backend's): K [kv][ctx][D]; V [kv][ctx/64][D][64] — transposed inside blocks of 64 keys, so a
//    P·V B tile is 8 consecutive keys of one dim and a chunk of keys is contiguous, like K's; int8 codes with f16
//    scales [kv][ctx], or BF16 values. Every chunk is two contiguous streams read with 16- and 8-byte loads. A
//    chunk is 64 keys (int8, D = 128) or 32 (BF16, or D = 256), sized so a wave holds one in registers and the next
//    in flight.
//  * gqa_decode: a workgroup of 4 waves per (KV head, key range[, row tile]) — 8 at head dim 128 with one row tile
//    on a long cache (one chunk per wave, two waves per SIMD). Each workgroup prepares its own query rows (q
//    RMSNorm, RoPE in registers, power-of-two prescale into F16: the MFMA B operand, in LDS); the workgroups whose
//    range holds the step's new tokens first quantize their keys and values into the cache. Each wave streams its
//    share of the range in chunks with the next chunk prefetched into registers. The rep·T query rows of the KV head
//    are A tiles of v_mfma_f32_16x16x32_f16; int8 codes become exact F16 with an XOR / byte-permute / packed
//    subtract; QKᵀ and P·V run on MFMA, the softmax online; the V scale folds into P (with a per-chunk power of two
//    so it stays in F16 range). The BF16 cache feeds v_mfma_f32_16x16x32_bf16 as it is (q, P and the cache are all
//    BF16-valued: the products are exact). The waves fold their (O, m, l) in LDS; the workgroup writes one partial.
//    With at most 16 partials per KV head the last workgroup to finish (a device-scope arrival counter) merges them
//    in group order and applies the gate.
//  * gqa_merge: otherwise, one wave per (head, token) folds the partials in key order and applies the gate —
//    deterministic either way.
#include "mi_common.h"

#include <algorithm>
#include <type_traits>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace {

constexpr int BLOCK = 64;       // keys per V block (the V codes are transposed inside it)
constexpr int TMAX = 16;
constexpr int DMAX = 256;

struct GqaArgs {
  int t, heads, kv, d, rot, pos, ctx, gate, qk_norm, rep, rows;
  int n_groups, group_len;                      // decode workgroups per KV head, keys per workgroup
  int xcd_tiles;                                // > 1: row tiles over workgroups in the XCD-grouped 1-D grid
  const uint16_t* proj; int ldp;
  const uint16_t* gsrc; int ldg;                // the gate rows in their own buffer (proj then holds q|k|v), or null
  const uint16_t* cosb; const uint16_t* sinb;   // [ctx][rot] BF16
  const float* q_norm; const float* k_norm;     // (1 + w), [D]
  float eps, scaling;
  void* kc; uint16_t* ks; void* vc; uint16_t* vs;   // int8 codes + f16 scales, or BF16 values (no scales)
  float* part_o; float* part_ml;                // [kv][group][rows][D], [kv][rows][group][2]
  uint32_t* cnt;                                // [kv] arrival counters (zero between calls) for the in-kernel merge
  uint16_t* qf; float* qsc;                     // gqa_prep's query rows [kv][64][D] (F16 prescaled, or BF16) and
                                                // their 2^p [kv][64]; null: each decode workgroup prepares its own
  int fmerge;                                   // 1: the last workgroup of a KV head to finish merges its partials
  uint16_t* y; int ldy;
  const int32_t* pos_dev;                       // device-resident position (a step program's StepState), or null
  const uint32_t* done;                         // the step state's stop flag, or null: set = append nothing
};

__device__ __forceinline__ bool stopped(const GqaArgs& a) { return a.done && *a.done; }

// the cache position of the step's first new token: the descriptor's, or the one a step program keeps on the device
__device__ __forceinline__ int cur_pos(const GqaArgs& a) { return a.pos_dev ? *a.pos_dev : a.pos; }

__device__ __forceinline__ float bfv(const uint16_t* p, long long i) { return bf16_bits_to_f32(p[i]); }

// 8 int8 codes (two dwords) → 8 exact F16 values
__device__ __forceinline__ f16x8 i8x8_to_f16(uint32_t lo, uint32_t hi) {
  const uint32_t magic = 0x64646464u;
  const uint32_t u0 = lo ^ 0x80808080u, u1 = hi ^ 0x80808080u;   // offset binary: c + 128
  union { uint32_t u; f16x2 h; } a, b, c, d;
  a.u = __builtin_amdgcn_perm(u0, magic, 0x00050004u);          // (1024 + u0, 1024 + u1)
  b.u = __builtin_amdgcn_perm(u0, magic, 0x00070006u);
  c.u = __builtin_amdgcn_perm(u1, magic, 0x00050004u);
  d.u = __builtin_amdgcn_perm(u1, magic, 0x00070006u);
  const f16x2 off = {(f16_t)1152.0f, (f16_t)1152.0f};
  const f16x2 x = a.h - off, y = b.h - off, z = c.h - off, w = d.h - off;
  return f16x8{x.x, x.y, y.x, y.y, z.x, z.y, w.x, w.y};
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// A q/k head vector's inputs, every one loaded before any is used (lane l: dims l + 64·u): the BF16 values, the
// norm weights, the RoPE cos / sin at the token's position (index clamped into the table past the rotary dims).
template <int DH>
struct HeadIn {
  float x[DH / 64], w[DH / 64], c[DH / 64], s[DH / 64];
};

__device__ float kZeros[DMAX];     // read in place of an absent table (norm weights, RoPE): the values go unused

template <int DH>
__device__ __forceinline__ void load_head(const GqaArgs& a, const uint16_t* src, const float* nw, int p, int lane,
                                          HeadIn<DH>& in) {
  // every load unconditional (a loaded value that meets a branch is waited for there): absent tables read zeros
  const float* wp = a.qk_norm ? nw : kZeros;
  const uint16_t* cp = a.rot > 0 ? a.cosb + (long long)p * a.rot : reinterpret_cast<const uint16_t*>(kZeros);
  const uint16_t* sp = a.rot > 0 ? a.sinb + (long long)p * a.rot : reinterpret_cast<const uint16_t*>(kZeros);
#pragma unroll
  for (int u = 0; u < DH / 64; ++u) {
    const int i = lane + 64 * u, ic = max(min(i, a.rot - 1), 0);
    in.x[u] = bfv(src, i);
    in.w[u] = wp[i];
    in.c[u] = bfv(cp, ic);
    in.s[u] = bfv(sp, ic);
  }
}

// The vector after the optional (1+w) RMSNorm and partial RoPE (BF16 values as f32), in the lane's registers
// (o[u]: dim lane + 64·u). RoPE pairs dim i with i ± rot/2: at rot/2 = 32 that is lane l ^ 32 of the same register (a
// lane swap), at a multiple of 64 the same lane's register u ± rot/128; other rotary widths go through tmp[D] (the
// wave's LDS scratch).
template <int DH>
__device__ __forceinline__ void norm_rope(const GqaArgs& a, const HeadIn<DH>& in, float (&o)[DH / 64], float* tmp,
                                          int lane) {
  constexpr int U = DH / 64;
  float x[U];
#pragma unroll
  for (int u = 0; u < U; ++u) x[u] = in.x[u];
  if (a.qk_norm) {
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) ss += x[u] * x[u];
    const float r = 1.0f / sqrtf(wave_sum(ss) / (float)DH + a.eps);
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = round_bf16((x[u] * r) * in.w[u]);
  }
  const int half = a.rot / 2;
  float pr[U];                                          // the partner dim's value
  if (half == 32) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x[u]), __float_as_int(x[u]), false, false);
      pr[u] = __int_as_float((lane & 32) ? r[0] : r[1]);
    }
  } else if ((half & 63) == 0) {
    const int sh = half >> 6;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float v = 0.0f;
#pragma unroll
      for (int q = 0; q < U; ++q) v = (q == u + sh || q == u - sh) && (q == u + sh) == (u < sh) ? x[q] : v;
      pr[u] = v;
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) tmp[lane + 64 * u] = x[u];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = lane + 64 * u;
      pr[u] = i < a.rot ? tmp[i < half ? i + half : i - half] : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = lane + 64 * u;
    if (i < a.rot) {
      const float rot = i < half ? -pr[u] : pr[u];
      o[u] = round_bf16(round_bf16(x[u] * in.c[u]) + round_bf16(rot * in.s[u]));
    } else {
      o[u] = x[u];
    }
  }
}

// store a BF16-valued vector (registers, dims lane + 64·u) as one cache row (wave cooperative): int8 codes at
// codes + stride·i and the f16 scale at *scale_out, or BF16 values at values + stride·i
template <int DH, bool BF>
__device__ __forceinline__ void store_row(const float (&x)[DH / 64], void* dst, long long stride, uint16_t* scale_out,
                                          int lane) {
  constexpr int U = DH / 64;
  if constexpr (BF) {
#pragma unroll
    for (int u = 0; u < U; ++u) static_cast<uint16_t*>(dst)[stride * (lane + 64 * u)] = f32_to_bf16_bits(x[u]);
  } else {
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) m = fmaxf(m, fabsf(x[u]));
    const float amax = wave_max(m);
    const f16_t sh = (f16_t)(amax / 127.0f);
    const float sc = (float)sh;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float c = sc > 0.0f ? fminf(fmaxf(rintf(x[u] / sc), -127.0f), 127.0f) : 0.0f;
      static_cast<int8_t*>(dst)[stride * (lane + 64 * u)] = (int8_t)(int)c;
    }
    if (lane == 0) *scale_out = __builtin_bit_cast(uint16_t, sh);
  }
}

constexpr int MAXROWS = 64;     // query rows per KV head (rep·T)
constexpr int kNW = 4;          // waves per decode workgroup (head dim 256; 128: gqa_waves())

__device__ __forceinline__ float pow2f(int e) { return __uint_as_float((uint32_t)(127 + e) << 23); }

__device__ __forceinline__ int prescale_exp(float mx) {   // 2^-p·mx in [2^14, 2^15): F16 keeps 11 bits of each value
  if (mx == 0.0f) return 0;
  const int p = (int)((__float_as_uint(mx) >> 23) & 0xFF) - 127 - 14;
  return min(max(p, -100), 100);
}

// Position of key k (0..63) inside its V block: the P·V MFMA sums over keys in any order, so the order is the one
// in which the score tile already holds them — lane (kg, m16) holds keys 16·kt + 4·kg + i of score tile kt, and as
// the B operand of k-block ks (keys 32·ks + …) its 8 values are tiles 2·ks, 2·ks + 1 — and those 8 keys sit
// together, with lane group kg's two k-blocks side by side (16 positions from 16·kg): one 16-byte load per lane
// and dim for a 64-key int8 chunk.
__device__ __forceinline__ int vblock_pos(int k) { return ((k & 15) >> 2) * 16 + (k >> 5) * 8 + ((k >> 4) & 1) * 4 + (k & 3); }

// Query row `row` of KV head j (row = token·rep + head within the group): its inputs (issued, not waited for).
template <int DH>
__device__ __forceinline__ void load_q(const GqaArgs& a, int j, int row, int pos, int lane, HeadIn<DH>& in) {
  const int q_cols = a.gate && !a.gsrc ? 2 * DH : DH;
  const int t = row / a.rep, h = j * a.rep + (row - t * a.rep);
  // a device position past the cache (a stopped program's queued steps) must not read past the RoPE tables
  load_head<DH>(a, a.proj + (long long)t * a.ldp + h * q_cols, a.q_norm, min(pos + t, a.ctx - 1), lane, in);
}

// The query row normed, roped and — int8 cache — prescaled by a power of two into F16 (exact above 2^-14 of the
// row's max; its 2^p to *sc), or BF16 as it is (the BF16 MFMA takes it exactly), into dst[D] (LDS); tmp[D]: the
// wave's LDS scratch.
template <int DH, bool BF>
__device__ void finish_q(const GqaArgs& a, const HeadIn<DH>& in, float* tmp, uint16_t* dst, float* sc, int lane) {
  constexpr int U = DH / 64;
  float o[U];
  norm_rope<DH>(a, in, o, tmp, lane);
  if constexpr (BF) {
#pragma unroll
    for (int u = 0; u < U; ++u) dst[lane + 64 * u] = f32_to_bf16_bits(o[u]);
    if (lane == 0) *sc = 1.0f;
  } else {
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) m = fmaxf(m, fabsf(o[u]));
    const int p = prescale_exp(wave_max(m));
    const float inv = pow2f(-p);
#pragma unroll
    for (int u = 0; u < U; ++u) dst[lane + 64 * u] = __builtin_bit_cast(uint16_t, (f16_t)(o[u] * inv));
    if (lane == 0) *sc = pow2f(p);
  }
}

// Token t's key and value rows of KV head j: their inputs (issued, not waited for).
template <int DH>
struct KvIn {
  HeadIn<DH> k;
  float v[DH / 64];
};
template <int DH>
__device__ __forceinline__ void load_kv(const GqaArgs& a, int j, int t, int pos, int lane, KvIn<DH>& in) {
  const int q_cols = a.gate && !a.gsrc ? 2 * DH : DH;
  const uint16_t* row = a.proj + (long long)t * a.ldp;
  load_head<DH>(a, row + a.heads * q_cols + j * DH, a.k_norm, min(pos + t, a.ctx - 1), lane, in.k);
  const uint16_t* v = row + a.heads * q_cols + a.kv * DH + j * DH;
#pragma unroll
  for (int u = 0; u < DH / 64; ++u) in.v[u] = bfv(v, lane + 64 * u);
}

// ... appended to the cache: the key normed and roped, both quantized to int8 codes + f16 scale (or stored as BF16)
template <int DH, bool BF>
__device__ void append_kv(const GqaArgs& a, int j, int t, int pos, const KvIn<DH>& in, float* tmp, int lane) {
  constexpr int U = DH / 64;
  const int p = pos + t;
  if (p >= a.ctx) return;                         // past the cache (a device position the host cannot check)
  constexpr int ES = BF ? 2 : 1;                  // bytes per cache element
  char* kc = static_cast<char*>(a.kc);
  char* vc = static_cast<char*>(a.vc);
  float k[U];
  norm_rope<DH>(a, in.k, k, tmp, lane);
  store_row<DH, BF>(k, kc + ((long long)j * a.ctx + p) * DH * ES, 1, a.ks ? a.ks + (long long)j * a.ctx + p : nullptr,
                    lane);
  store_row<DH, BF>(in.v, vc + (((long long)j * a.ctx + (p & ~(BLOCK - 1))) * DH + vblock_pos(p & (BLOCK - 1))) * ES,
                    BLOCK, a.vs ? a.vs + (long long)j * a.ctx + p : nullptr, lane);
}

// The separate preparation launch, where in-workgroup preparation would cost more than a launch (many rows per
// workgroup, or more workgroups than one round of CUs): one wave per (head or KV head, token) — a query row into
// the workspace, or a token's key and value into the cache.
template <int DH, bool BF>
__global__ __launch_bounds__(64) void gqa_prep(GqaArgs a) {
  __shared__ float tmp[DH];
  const int lane = threadIdx.x, x = blockIdx.x, t = blockIdx.y;
  if (stopped(a)) return;
  const int pos = cur_pos(a);
  if (x < a.heads) {
    const int j = x / a.rep, row = t * a.rep + (x - j * a.rep);
    HeadIn<DH> in;
    load_q<DH>(a, j, row, pos, lane, in);
    finish_q<DH, BF>(a, in, tmp, a.qf + ((long long)j * MAXROWS + row) * DH, a.qsc + j * MAXROWS + row, lane);
  } else {
    KvIn<DH> in;
    load_kv<DH>(a, x - a.heads, t, pos, lane, in);
    append_kv<DH, BF>(a, x - a.heads, t, pos, in, tmp, lane);
  }
}

// ---- device-scope (coherent across the XCDs' L2s) partial stores and loads, for the in-kernel merge -------------
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev2(float* p, float x, float y) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p),
                     (unsigned long long)__float_as_uint(x) | ((unsigned long long)__float_as_uint(y) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev4(float* p, f32x4 v) {
  auto* q = reinterpret_cast<unsigned long long*>(p);
  __hip_atomic_store(q, (unsigned long long)__float_as_uint(v[0]) | ((unsigned long long)__float_as_uint(v[1]) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, (unsigned long long)__float_as_uint(v[2]) | ((unsigned long long)__float_as_uint(v[3]) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_dev2(const float* p) {
  return __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float lo_f(unsigned long long u) { return __uint_as_float((uint32_t)u); }
__device__ __forceinline__ float hi_f(unsigned long long u) { return __uint_as_float((uint32_t)(u >> 32)); }

// The merge of KV head j's partials inside the decode launch, by the workgroup that finished last: each half-wave
// takes rows hr, hr + 2·NW, … (lane: E = D/32 dims, the pairs 64·e + 2·lane + {0, 1}, so an 8-byte load
// instruction reads 256 contiguous bytes); per row the common max and the weights over the groups (lane g holds
// group g's (m, l)), l by a fixed-order half-wave sum, O in group order with every group's partial in flight at
// once (G ≤ MG); normalize, BF16, × bf16(σ(gate)) — deterministic. The partials are read with device-scope loads:
// they were written from other XCDs. Instruction count matters here: one wave per SIMD issues a vector instruction
// every 4 cycles, so the loop carries no division and no per-item address arithmetic beyond one add.
constexpr int MG = 16;          // groups the in-kernel merge takes (more: the gqa_merge launch)
bool merge_fits(int n_groups, int rows, int nw) { return n_groups <= MG && rows <= 4 * nw; }

template <int DH, int NW>
__device__ void merge_head(const GqaArgs& a, int j, int w, int lane) {
  constexpr int E = DH / 32, E2 = E / 2;          // dims per lane, in 8-byte loads
  const int G = a.n_groups, hl = lane & 31, hw = lane >> 5;
  for (int row = 2 * w + hw; row < a.rows; row += 2 * NW) {     // the two halves of a wave may end apart
    const int t = row / a.rep, h = j * a.rep + (row - t * a.rep);
    const uint16_t* gp = a.gsrc ? a.gsrc + (long long)t * a.ldg + h * DH
                                : a.proj + (long long)t * a.ldp + (a.gate ? h * 2 * DH + DH : 0);
    const float* po = a.part_o + ((long long)j * G * a.rows + row) * DH + 2 * hl;   // group g at + g·rows·D
    const long long gstride = (long long)a.rows * DH;
    unsigned long long it[MG][E2];
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
      for (int e = 0; e < E2; ++e) it[g][e] = g < G ? ld_dev2(po + g * gstride + 64 * e) : 0ull;
    const unsigned long long mlv = hl < G ? ld_dev2(a.part_ml + ((long long)(j * a.rows + row) * G + hl) * 2)
                                          : 0xFF800000ull;      // (m, l) = (-inf, 0)
    uint32_t gb[E2];                                            // the gate's BF16 pairs
#pragma unroll
    for (int e = 0; e < E2; ++e) gb[e] = *reinterpret_cast<const uint32_t*>(gp + 64 * e + 2 * hl);
    const float m = lo_f(mlv);
    const float M = max_xor16(max16(m));
    const float wl = m == -INFINITY ? 0.0f : __expf(m - M);
    const float l = add_xor16(sum16(wl * hi_f(mlv)));
    float o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
#pragma unroll
    for (int g = 0; g < MG; ++g) {
      // group g's weight from lane g of this half (the two halves hold different rows)
      const float wa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), g));
      const float wb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), 32 + g));
      const float wg = hw ? wb : wa;
#pragma unroll
      for (int e = 0; e < E2; ++e) {
        o[2 * e] += wg * lo_f(it[g][e]);
        o[2 * e + 1] += wg * hi_f(it[g][e]);
      }
    }
    uint16_t* yp = a.y + (long long)t * a.ldy + h * DH + 2 * hl;
#pragma unroll
    for (int e = 0; e < E2; ++e) {
      float y0 = round_bf16(o[2 * e] / l), y1 = round_bf16(o[2 * e + 1] / l);
      if (a.gate) {
        y0 = round_bf16(y0 * round_bf16(1.0f / (1.0f + __expf(-bf16_bits_to_f32((uint16_t)(gb[e] & 0xFFFF))))));
        y1 = round_bf16(y1 * round_bf16(1.0f / (1.0f + __expf(-bf16_bits_to_f32((uint16_t)(gb[e] >> 16))))));
      }
      *reinterpret_cast<uint32_t*>(yp + 64 * e) = f32_to_bf16_bits(y0) | ((uint32_t)f32_to_bf16_bits(y1) << 16);
    }
  }
}

// The geometry of one decode instantiation: head dim DH, cache element type (BF: BF16, else int8 codes + scales).
template <int DH, bool BF>
struct Geo {
  static constexpr int CH = (!BF && DH == 128) ? 64 : 32;   // keys per chunk
  static constexpr int KT = CH / 16;                          // score tiles per chunk
  static constexpr int KS = CH / 32;                          // P·V k-blocks per chunk
  static constexpr int NS = DH / 32;                          // QKᵀ k-blocks per score tile
  static constexpr int NC = DH / 16;                          // O column tiles
  static constexpr int KW = BF ? NS : NS / 2;                 // 16-byte K loads per key and lane
  static constexpr int VW = BF ? 4 : 2;                       // dwords of V per (k-block, column tile) and lane
};

// a chunk as this lane holds it: K of key k0 + 16·kt + m16, dims (DH/4)·kg + [0, DH/4); the scales of keys
// k0 + 16·kt + 4·kg + [0, 4) (int8); V of dim 16·ct + m16, keys (block order) 32·ks + 8·kg + [0, 8)
template <int DH, bool BF>
struct Chunk {
  using G = Geo<DH, BF>;
  uint4 k[G::KT][G::KW];
  uint2 ksc[BF ? 1 : G::KT], vsc[BF ? 1 : G::KT];
  uint32_t v[G::KS][G::NC][G::VW];
};

template <int DH, bool BF>
__device__ __forceinline__ void load_k(const GqaArgs& a, int j, int k0, int m16, int kg, Chunk<DH, BF>& c) {
  using G = Geo<DH, BF>;
  constexpr int ES = BF ? 2 : 1;
  const char* kb = static_cast<const char*>(a.kc) + (long long)j * a.ctx * DH * ES;
#pragma unroll
  for (int kt = 0; kt < G::KT; ++kt) {
    const char* kp = kb + ((long long)(k0 + kt * 16 + m16) * DH + (DH / 4) * kg) * ES;
#pragma unroll
    for (int w = 0; w < G::KW; ++w) c.k[kt][w] = *reinterpret_cast<const uint4*>(kp + 16 * w);
    if constexpr (!BF) {
      c.ksc[kt] = *reinterpret_cast<const uint2*>(a.ks + (long long)j * a.ctx + k0 + kt * 16 + 4 * kg);
      c.vsc[kt] = *reinterpret_cast<const uint2*>(a.vs + (long long)j * a.ctx + k0 + kt * 16 + 4 * kg);
    }
  }
}

template <int DH, bool BF>
__device__ __forceinline__ void load_v(const GqaArgs& a, int j, int k0, int m16, int kg, Chunk<DH, BF>& c) {
  using G = Geo<DH, BF>;
  constexpr int ES = BF ? 2 : 1;
  // the chunk's keys in their V block (block k0 / 64): lane group kg's 8 keys of k-block ks of a chunk starting at
  // key 32·h of the block sit at positions 16·kg + 8·(h + ks)
  const char* vp = static_cast<const char*>(a.vc) +
                   (((long long)j * a.ctx + (k0 & ~(BLOCK - 1))) * DH + 16 * kg + 8 * ((k0 & (BLOCK - 1)) >> 5)) * ES;
  if constexpr (!BF && G::KS == 2) {            // both k-blocks in one 16-byte load
#pragma unroll
    for (int ct = 0; ct < G::NC; ++ct) {
      const uint4 u = *reinterpret_cast<const uint4*>(vp + (long long)(ct * 16 + m16) * BLOCK);
      c.v[0][ct][0] = u.x; c.v[0][ct][1] = u.y; c.v[1][ct][0] = u.z; c.v[1][ct][1] = u.w;
    }
    return;
  }
#pragma unroll
  for (int ks = 0; ks < G::KS; ++ks)
#pragma unroll
    for (int ct = 0; ct < G::NC; ++ct) {
      const char* q = vp + ((long long)(ct * 16 + m16) * BLOCK + ks * 8) * ES;
      if constexpr (BF) {
        const uint4 u = *reinterpret_cast<const uint4*>(q);
        c.v[ks][ct][0] = u.x; c.v[ks][ct][1] = u.y; c.v[ks][ct][2] = u.z; c.v[ks][ct][3] = u.w;
      } else {
        const uint2 u = *reinterpret_cast<const uint2*>(q);
        c.v[ks][ct][0] = u.x; c.v[ks][ct][1] = u.y;
      }
    }
}

__device__ __forceinline__ float f16_lo(uint32_t u) { return (float)__builtin_bit_cast(f16_t, (uint16_t)(u & 0xFFFF)); }
__device__ __forceinline__ float f16_hi(uint32_t u) { return (float)__builtin_bit_cast(f16_t, (uint16_t)(u >> 16)); }

// The decode workgroup: NW waves over one key range of KV head j. Everything is computed transposed so that a
// lane owns one query row (row = 16·rt + m16): Sᵀ = K·Qᵀ (A = the K tile, B = the query rows), softmax over the
// lane's keys plus the lanes l ^ 16, l ^ 32, l ^ 48 of the same row, and Oᵀ += Vᵀ·Pᵀ with Pᵀ straight from the score
// registers (no LDS round trip) — every per-row quantity is lane-local.
template <int RT, int DH, bool BF, int NW, bool OWN>
__global__ __launch_bounds__(64 * NW, 1) void gqa_decode(GqaArgs a) {
  using G = Geo<DH, BF>;
  using OpT = typename std::conditional<BF, bf16x8, f16x8>::type;
  constexpr int CH = G::CH;
  // one row tile at head dim 128: the waves' O meet in a pairwise tree through per-wave slabs (wave w > 0 owns slab
  // w - 1); otherwise they are summed into red one wave after another
  constexpr bool TREE = RT == 1 && DH == 128;
  __shared__ __attribute__((aligned(16))) float red[TREE ? 1 : RT * 16][DH + 4];   // the workgroup's O, row-major
  __shared__ __attribute__((aligned(16))) float slab[TREE ? NW - 1 : 1][16][DH + 4];
  __shared__ float mls[NW][RT * 16][2];
  __shared__ __attribute__((aligned(16))) uint16_t qs[RT * 16][DH];   // the workgroup's query rows (B operands)
  __shared__ float qss[RT * 16];                                      // their 2^p (int8 cache)
  __shared__ float ptmp[NW][DH];                                      // each wave's scratch for the row preparation
  __shared__ uint32_t last_in;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: the key range is a scalar loop
  // the workgroup's (key range g, KV head j, row-tile group zt): from the grid, or — row tiles spread over
  // workgroups (a.xcd_tiles = their number) — from a 1-D grid in which the tiles of one key range take dispatch
  // slots 8 apart: consecutive workgroups go to the 8 XCDs in turn, so the range's tiles run together on one XCD
  // and all but the first read the range from that XCD's L2
  int g = blockIdx.x, j = blockIdx.y, zt = blockIdx.z;
  if (a.xcd_tiles > 1) {
    const int id = blockIdx.x, slot = id >> 3;
    zt = slot % a.xcd_tiles;
    const int r = (slot / a.xcd_tiles) * 8 + (id & 7);           // key range × KV head
    if (r >= a.n_groups * a.kv) return;                          // grid padding: workgroup-uniform
    g = r % a.n_groups;
    j = r / a.n_groups;
  }
  if (stopped(a)) return;                               // workgroup-uniform
  const int pos = cur_pos(a);
  const int n_keys = min(pos + a.t, a.ctx);
  const int kb = g * a.group_len;
  // the last group also takes the new tokens; with a device position the groups cover the planned bound and the
  // ones past the position are empty (their partials fold in with weight 0)
  const int ke = g == a.n_groups - 1 ? n_keys : min(kb + a.group_len, n_keys);
  const int nch = max(0, (ke - kb + CH - 1) / CH);
  // Where the registers allow (VA), two chunks in flight per wave (see below). Otherwise, with chunks shorter than a
  // V block (BF16 cache, or head dim 256), the waves take the range's chunks in turn (wave w: chunks w, w + NW, …):
  // a 32-key chunk reads half of each 128-byte line of its V block, and the block's two chunks, on neighbouring
  // waves, then request the same lines together — one chunk after the other in one wave, the line had often left
  // the L2 before its second half was read (head dim 256, 32K, M = 1: 1.27 × the range's bytes fetched).
  constexpr bool VA = NW == 4 && DH == 128 && (RT <= 2 || (RT == 3 && BF));   // two chunks: at most 48 loads in flight
  constexpr bool STRIDE = !VA && CH < BLOCK;
  const int k_begin = STRIDE ? kb + w * CH : kb + (w * nch / NW) * CH;
  const int k_end = STRIDE ? ke : min(ke, kb + ((w + 1) * nch / NW) * CH);
  constexpr int K_STEP = STRIDE ? NW * CH : CH;         // from one of the wave's chunks to the next
  const int m16 = lane & 15, kg = lane >> 4;

  const int r0 = zt * RT * 16;                          // this workgroup's first query row
  const int nrows = min(RT * 16, a.rows - r0);
  // OWN: the query rows are prepared in every workgroup (norm, RoPE, prescale: a few hundred bytes of input per row);
  // the workgroups whose key range holds new tokens first append the tokens' keys and values to the cache (the same
  // bytes in every such workgroup; the tokens spread over the waves), so that their own reads of the range see
  // them. The wave's query rows (at most 16) have their inputs issued ahead of the chunk loads, and are finished
  // while those are in flight. (Appending by the one wave whose keys they are, with no workgroup barrier, measured
  // slower: 4K M = 1 13.0 vs 12.3 µs, M = 8 20.9 vs 15.1 µs.) Otherwise gqa_prep ran first: the rows come from its
  // workspace and the cache already holds the new tokens.
  constexpr int QB = (RT * 16 + NW - 1) / NW;
  static_assert(QB <= 16, "a wave prepares at most 16 query rows");
  constexpr bool own = OWN;                             // the rows (and the append) are this launch's, or gqa_prep's
  HeadIn<DH> qin[own ? QB : 1];
  // the query rows as B tiles (k-permuted: lane holds dims (DH/4)·kg + 8·s + i of row r0 + 16·rt + m16), zero past
  // rows: from LDS once this workgroup has prepared them, or straight from gqa_prep's workspace
  OpT qb[RT][G::NS];
  float rsc[RT];                                        // the lane's row: 2^p of its prescale (int8 cache)
  int qlim[RT];                                         // the lane's row: last key it may see (causal)
  if constexpr (own) {
#pragma unroll
    for (int i = 0; i < QB; ++i) load_q<DH>(a, j, r0 + min(w + NW * i, nrows - 1), pos, lane, qin[i]);
  } else {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = r0 + rt * 16 + m16;
      const bool ok = row < a.rows;
      const uint16_t* src = a.qf + ((long long)j * MAXROWS + (ok ? row : 0)) * DH + (DH / 4) * kg;
#pragma unroll
      for (int s = 0; s < G::NS; ++s) {
        const uint4 u = *reinterpret_cast<const uint4*>(src + 8 * s);
        qb[rt][s] = __builtin_bit_cast(OpT, ok ? u : uint4{0u, 0u, 0u, 0u});
      }
      rsc[rt] = ok ? a.qsc[j * MAXROWS + row] : 1.0f;
      qlim[rt] = ok ? pos + row / a.rep : n_keys;       // rows past `rows` hold q = 0: finite, never written
    }
  }
  if (own && kb < n_keys && ke > pos) {                 // workgroup-uniform: the range holds new tokens
    constexpr int AT = (TMAX + NW - 1) / NW;          // tokens a wave appends: their inputs loaded together
    KvIn<DH> kin[AT];
#pragma unroll
    for (int i = 0; i < AT; ++i) load_kv<DH>(a, j, min(w + NW * i, a.t - 1), pos, lane, kin[i]);
#pragma unroll
    for (int i = 0; i < AT; ++i)
      if (w + NW * i < a.t) append_kv<DH, BF>(a, j, w + NW * i, pos, kin[i], ptmp[w], lane);
    __syncthreads();                                    // the appended rows visible to every wave of the workgroup
  }
  // Where the registers allow (VA), two chunks in flight: buffer A holds chunks k_begin, k_begin + 2·CH, …, B the
  // ones between, each chunk's K and V loaded one chunk ahead; otherwise each chunk is loaded as it starts.
  // Every load is issued whether or not its chunk exists (a chunk past the wave's range re-reads the last one in
  // range, or the range's start when it is empty — chunks lie inside the cache: ctx % 64 == 0), after the query
  // rows, so the in-order memory counter lets a chunk's wait leave the other chunk's loads outstanding.
  Chunk<DH, BF> ca, cb;
  const int k_last = k_begin < k_end ? k_begin + ((k_end - 1 - k_begin) / K_STEP) * K_STEP : min(k_begin, a.ctx - CH);
  auto load_chunk = [&](Chunk<DH, BF>& c, int k0) {
    const int kk = min(k0, k_last);
    load_k<DH, BF>(a, j, kk, m16, kg, c);
    load_v<DH, BF>(a, j, kk, m16, kg, c);
    __builtin_amdgcn_sched_barrier(0);                // the loads stay here, ahead of the chunk's math
  };
  // the wave's first chunk in flight while the query rows are prepared; the second (if the wave has one) is issued
  // after them, so the rows' waits never cover the chunk loads. With more than one row tile the rows and a chunk do
  // not fit the registers together: the rows are finished first.
  constexpr bool QFIRST = RT > 1;
  if constexpr (VA && !QFIRST) load_chunk(ca, k_begin);
  // head dim 256 (no second buffer) still issues its first chunk here, ahead of the rows' preparation, and loads the
  // later ones as they start: the reference geometry at 32K, M = 1 41.5 → 39.8 µs. (The 8-wave head-dim-128 kernel
  // measured slower so: 18.0 → 19.2 µs at 32K.)
  constexpr bool PRE1 = !VA && RT == 1 && DH == 256;
  if constexpr (PRE1) load_chunk(ca, k_begin);
  if constexpr (own) {
#pragma unroll
    for (int i = 0; i < QB; ++i) {
      const int r = w + NW * i;
      if (r < nrows) finish_q<DH, BF>(a, qin[i], ptmp[w], qs[r], &qss[r], lane);
    }
  }
  if constexpr (VA && QFIRST) load_chunk(ca, k_begin);
  if constexpr (own) {
    lds_barrier();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int lr = rt * 16 + m16, row = r0 + lr;
      const bool ok = row < a.rows;
      const uint16_t* src = &qs[ok ? lr : 0][(DH / 4) * kg];
#pragma unroll
      for (int s = 0; s < G::NS; ++s) {
        const uint4 u = *reinterpret_cast<const uint4*>(src + 8 * s);
        qb[rt][s] = __builtin_bit_cast(OpT, ok ? u : uint4{0u, 0u, 0u, 0u});
      }
      rsc[rt] = ok ? qss[lr] : 1.0f;
      qlim[rt] = ok ? pos + row / a.rep : n_keys;         // rows past `rows` hold q = 0: finite, never written
    }
  }

  f32x4 o[RT][G::NC];                                   // o[rt][ct][i] = O[row 16·rt + m16][dim 16·ct + 4·kg + i]
  float m_run[RT], l_run[RT];                           // l_run: this lane's share (its keys per chunk)
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int ct = 0; ct < G::NC; ++ct) o[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.0f;
  }
  int pv_cur = 0;                                       // O is held in units of 2^pv_cur (int8 cache)

  auto process = [&](Chunk<DH, BF>& cur, int k0) {
    if constexpr (!VA) {                              // no registers for a second chunk: load this one now
      if (!PRE1 || k0 != k_begin) {                   // (the first one was issued ahead)
        load_k<DH, BF>(a, j, min(k0, k_last), m16, kg, cur);
        load_v<DH, BF>(a, j, min(k0, k_last), m16, kg, cur);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const bool full = k0 + CH <= k_end && k0 + CH - 1 <= pos;     // every key valid and visible to every row
    float ksc[G::KT][4], vsc[G::KT][4];
    int pv = pv_cur;
    float resc = 1.0f;
    if constexpr (!BF) {
      float vmax = 0.0f;
#pragma unroll
      for (int kt = 0; kt < G::KT; ++kt) {
        const uint2 kq = cur.ksc[kt], vq = cur.vsc[kt];
        ksc[kt][0] = f16_lo(kq.x); ksc[kt][1] = f16_hi(kq.x); ksc[kt][2] = f16_lo(kq.y); ksc[kt][3] = f16_hi(kq.y);
        vsc[kt][0] = f16_lo(vq.x); vsc[kt][1] = f16_hi(vq.x); vsc[kt][2] = f16_lo(vq.y); vsc[kt][3] = f16_hi(vq.y);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (!full && k0 + kt * 16 + 4 * kg + i >= k_end) vsc[kt][i] = 0.0f;
          vmax = fmaxf(vmax, vsc[kt][i]);
        }
      }
      vmax = max_xor32(max_xor16(vmax));
      // the chunk's V-scale prescale 2^-pv keeps P'' = p·v_scale·2^-pv in F16 range
      pv = vmax == 0.0f ? pv_cur : prescale_exp(vmax);
      const float pv_inv = pow2f(-pv);
      resc = pow2f(pv_cur - pv);
#pragma unroll
      for (int kt = 0; kt < G::KT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) vsc[kt][i] *= pv_inv;
    }

    OpT ka[G::KT][G::NS];                               // the K tiles as MFMA A operands
#pragma unroll
    for (int kt = 0; kt < G::KT; ++kt)
#pragma unroll
      for (int s = 0; s < G::NS; ++s) {
        if constexpr (BF) {
          ka[kt][s] = as_bf16x8(cur.k[kt][s]);
        } else {
          const uint4 u = cur.k[kt][s / 2];
          ka[kt][s] = (s & 1) ? i8x8_to_f16(u.z, u.w) : i8x8_to_f16(u.x, u.y);
        }
      }
    OpT pb[RT][G::KS];                                  // Pᵀ B tiles: element i of k-block ks = key tile 2·ks + i/4
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float sc[G::KT][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < G::KT; ++kt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < G::NS; ++s) {
          if constexpr (BF) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kt][s], qb[rt][s], acc, 0, 0, 0);
          else acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt][s], qb[rt][s], acc, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v;
          if constexpr (BF) v = round_bf16(round_bf16(acc[i]) * a.scaling);
          else v = round_bf16(round_bf16(acc[i] * (rsc[rt] * ksc[kt][i])) * a.scaling);
          if (!full) {
            const int key = k0 + kt * 16 + 4 * kg + i;
            v = (key < k_end && key <= qlim[rt]) ? v : -INFINITY;
          }
          sc[kt][i] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = max_xor32(max_xor16(mx));
      const float mnew = fmaxf(m_run[rt], mx);
      const float alpha = m_run[rt] == -INFINITY ? 0.0f : __expf(m_run[rt] - mnew);
      float psum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < G::KT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = sc[kt][i] == -INFINITY ? 0.0f : __expf(sc[kt][i] - mnew);
          psum += p;
          if constexpr (BF) pb[rt][kt >> 1][(kt & 1) * 4 + i] = (__bf16)p;
          else pb[rt][kt >> 1][(kt & 1) * 4 + i] = (f16_t)(round_bf16(p) * vsc[kt][i]);
        }
      l_run[rt] = l_run[rt] * alpha + psum;
      m_run[rt] = mnew;
      const float f = alpha * resc;
#pragma unroll
      for (int ct = 0; ct < G::NC; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[rt][ct][i] *= f;
    }
    pv_cur = pv;
    // Oᵀ += Vᵀ·Pᵀ
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks)
#pragma unroll
      for (int ct = 0; ct < G::NC; ++ct) {
        if constexpr (BF) {
          const bf16x8 va = as_bf16x8(uint4{cur.v[ks][ct][0], cur.v[ks][ct][1], cur.v[ks][ct][2], cur.v[ks][ct][3]});
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            o[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[rt][ks], o[rt][ct], 0, 0, 0);
        } else {
          const f16x8 va = i8x8_to_f16(cur.v[ks][ct][0], cur.v[ks][ct][1]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            o[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[rt][ks], o[rt][ct], 0, 0, 0);
        }
      }
  };
  // head dim 128, one row tile: the first two chunks straight-line (all of a wave's range up to 32K keys, where the
  // compiler's waits are exact; in the loop the waits of the chunk at its head drain both buffers), the rest in the
  // loop. Larger geometries do not have the registers for the extra copies of the chunk code.
  constexpr bool SL = RT == 1 && DH == 128;
  // A wave with one chunk (every wave up to 32K keys at 4 KV heads) issues no other loads: a load left in flight
  // past the last chunk is waited for where its registers are reused, one more memory round trip on the way out.
  if constexpr (!VA) {
    for (int k0 = k_begin; k0 < k_end; k0 += K_STEP) process(ca, k0);
  } else if (k_begin + CH >= k_end) {
    if (k_begin < k_end) process(ca, k_begin);
  } else if (!SL) {
    load_chunk(cb, k_begin + CH);
    for (int k0 = k_begin; k0 < k_end; k0 += 2 * CH) {
      process(ca, k0);
      load_chunk(ca, k0 + 2 * CH);
      if (k0 + CH >= k_end) break;
      process(cb, k0 + CH);
      load_chunk(cb, k0 + 3 * CH);
    }
  } else {
    load_chunk(cb, k_begin + CH);
    process(ca, k_begin);
    load_chunk(ca, k_begin + 2 * CH);
    if (k_begin + CH < k_end) {
      process(cb, k_begin + CH);
      load_chunk(cb, k_begin + 3 * CH);
      for (int k0 = k_begin + 2 * CH; k0 < k_end; k0 += 2 * CH) {
        process(ca, k0);
        load_chunk(ca, k0 + 2 * CH);
        if (k0 + CH >= k_end) break;
        process(cb, k0 + CH);
        load_chunk(cb, k0 + 3 * CH);
      }
    }
  }

  // ---- fold the workgroup's waves: common max, O summed in LDS (a pairwise tree, or in wave order), one partial per
  // workgroup ----------------------------------------------------------------------------------------------------
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float l = quad16_sum(l_run[rt]);
    if (kg == 0) {
      mls[w][rt * 16 + m16][0] = m_run[rt];
      mls[w][rt * 16 + m16][1] = l;
    }
  }
  lds_barrier();
  const float unscale = pow2f(pv_cur);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = rt * 16 + m16;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, mls[ww][row][0]);
    const float f = m_run[rt] == -INFINITY ? 0.0f : __expf(m_run[rt] - M) * unscale;
#pragma unroll
    for (int ct = 0; ct < G::NC; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[rt][ct][i] *= f;
  }
  const long long base = ((long long)j * a.n_groups + g) * a.rows + r0;
  if constexpr (TREE) {
    // step `half`: waves [half, 2·half) publish their O, waves [0, half) add it (wave r takes wave r + half); the
    // slabs a step writes were not read in the step before, so one barrier per step. A fixed order: deterministic.
    for (int half = NW / 2; half >= 1; half >>= 1) {
      if (w >= half && w < 2 * half) {
#pragma unroll
        for (int ct = 0; ct < G::NC; ++ct)
          *reinterpret_cast<f32x4*>(&slab[w - 1][m16][ct * 16 + 4 * kg]) = o[0][ct];
      }
      lds_barrier();
      if (w < half) {
#pragma unroll
        for (int ct = 0; ct < G::NC; ++ct)
          o[0][ct] += *reinterpret_cast<const f32x4*>(&slab[w + half - 1][m16][ct * 16 + 4 * kg]);
      }
    }
    if (w == 0 && m16 < nrows) {                        // wave 0 holds the workgroup's O: straight to its partial
#pragma unroll
      for (int ct = 0; ct < G::NC; ++ct) {
        float* dst = a.part_o + (base + m16) * DH + ct * 16 + 4 * kg;
        if (a.fmerge) st_dev4(dst, o[0][ct]);
        else *reinterpret_cast<f32x4*>(dst) = o[0][ct];
      }
    }
  } else {
    for (int ww = 0; ww < NW; ++ww) {
      if (w == ww) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int ct = 0; ct < G::NC; ++ct) {
            f32x4* dst = reinterpret_cast<f32x4*>(&red[rt * 16 + m16][ct * 16 + 4 * kg]);
            *dst = ww == 0 ? o[rt][ct] : *dst + o[rt][ct];
          }
      }
      lds_barrier();
    }
    for (int idx = threadIdx.x; idx < nrows * DH; idx += 64 * NW) {
      if (a.fmerge) st_dev(a.part_o + base * DH + idx, red[idx / DH][idx % DH]);
      else a.part_o[base * DH + idx] = red[idx / DH][idx % DH];
    }
  }
  for (int row = threadIdx.x; row < nrows; row += 64 * NW) {
    float M = -INFINITY, L = 0.0f;
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, mls[ww][row][0]);
    for (int ww = 0; ww < NW; ++ww)
      if (mls[ww][row][0] != -INFINITY) L += __expf(mls[ww][row][0] - M) * mls[ww][row][1];
    if (a.fmerge) {
      st_dev2(a.part_ml + ((long long)(j * a.rows + r0 + row) * a.n_groups + g) * 2, M, L);
    } else {
      a.part_ml[((long long)(j * a.rows + r0 + row) * a.n_groups + g) * 2] = M;
      a.part_ml[((long long)(j * a.rows + r0 + row) * a.n_groups + g) * 2 + 1] = L;
    }
  }
  if (!a.fmerge) return;
  // The in-kernel merge: the partial's device-scope stores acknowledged (every wave), then one arrival on the KV
  // head's counter; the workgroup that brings it to the head's workgroup count merges and re-arms it. No fence: the
  // stores were performed at the device's coherence point before the count moved, and the merge reads there.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t total = (uint32_t)(a.n_groups * max(1, a.xcd_tiles));
    const uint32_t prev = __hip_atomic_fetch_add(a.cnt + j, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_in = prev == total - 1;
    if (prev == total - 1) __hip_atomic_store(a.cnt + j, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  lds_barrier();
  if (last_in) merge_head<DH, NW>(a, j, w, lane);
}

// one workgroup of MW waves per (query head, token): wave w folds partials w, w + MW, … (all its loads in flight
// at once), then wave 0 adds the MW sums in wave order — deterministic; normalize, BF16, × bf16(σ(gate))
constexpr int MW = 8;
template <int DH>
__global__ __launch_bounds__(64 * MW) void gqa_merge(GqaArgs a) {
  constexpr int U = DH / 64;
  constexpr int GB = 8;                                     // partials a wave holds at once (the one-pass form)
  __shared__ float red[MW][DH + 1];
  __shared__ float mxs[MW];
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (stopped(a)) return;
  const int j = h / a.rep;
  const int row = t * a.rep + (h - j * a.rep);
  const long long b0 = (long long)j * a.n_groups * a.rows + row;      // partial g at b0 + g·rows
  const long long mb = (long long)(j * a.rows + row) * a.n_groups;     // its (m, l) at mb + g
  // the gate first (an independent load; without a gate the row's first values are read and unused)
  const uint16_t* gp = a.gsrc ? a.gsrc + (long long)t * a.ldg + h * DH
                              : a.proj + (long long)t * a.ldp + (a.gate ? h * 2 * DH + DH : 0);
  float gv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) gv[u] = bfv(gp, lane + 64 * u);
  float M = -INFINITY, l = 0.0f, o[U];
#pragma unroll
  for (int u = 0; u < U; ++u) o[u] = 0.0f;
  if (a.n_groups <= MW * GB) {
    // one pass: every partial of the wave (groups w, w + MW, …; past the last, the last again with weight 0) in
    // flight at once, then the common max and the weighted sums in group order
    float pm[GB], pl[GB], po[GB][U];
#pragma unroll
    for (int i = 0; i < GB; ++i) {
      const long long b = b0 + (long long)min(w + MW * i, a.n_groups - 1) * a.rows;
      const long long bm = mb + min(w + MW * i, a.n_groups - 1);
      pm[i] = a.part_ml[bm * 2];
      pl[i] = a.part_ml[bm * 2 + 1];
#pragma unroll
      for (int u = 0; u < U; ++u) po[i][u] = a.part_o[b * DH + lane + 64 * u];
    }
    __builtin_amdgcn_sched_barrier(0);                        // all of them issued before the first wait
    float mw = -INFINITY;
#pragma unroll
    for (int i = 0; i < GB; ++i)
      if (w + MW * i < a.n_groups) mw = fmaxf(mw, pm[i]);
    if (lane == 0) mxs[w] = mw;
    __syncthreads();
#pragma unroll
    for (int ww = 0; ww < MW; ++ww) M = fmaxf(M, mxs[ww]);
#pragma unroll
    for (int i = 0; i < GB; ++i) {
      if (w + MW * i >= a.n_groups) break;
      const float wgt = pm[i] == -INFINITY ? 0.0f : __expf(pm[i] - M);
      l += wgt * pl[i];
#pragma unroll
      for (int u = 0; u < U; ++u) o[u] += wgt * po[i][u];
    }
  } else {
    for (int g = lane; g < a.n_groups; g += 64) M = fmaxf(M, a.part_ml[(mb + g) * 2]);
    M = wave_max(M);
#pragma unroll 8
    for (int g = w; g < a.n_groups; g += MW) {
      const long long b = b0 + (long long)g * a.rows;
      const float m = a.part_ml[(mb + g) * 2], lg = a.part_ml[(mb + g) * 2 + 1];
      const float wgt = m == -INFINITY ? 0.0f : __expf(m - M);
      l += wgt * lg;
#pragma unroll
      for (int u = 0; u < U; ++u) o[u] += wgt * a.part_o[b * DH + lane + 64 * u];
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) red[w][lane + 64 * u] = o[u];
  if (lane == 0) red[w][DH] = l;
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int u = 0; u < U; ++u) o[u] = red[0][lane + 64 * u];
  l = red[0][DH];
#pragma unroll
  for (int ww = 1; ww < MW; ++ww) {
#pragma unroll
    for (int u = 0; u < U; ++u) o[u] += red[ww][lane + 64 * u];
    l += red[ww][DH];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float y = round_bf16(o[u] / l);
    if (a.gate) y = round_bf16(y * round_bf16(1.0f / (1.0f + __expf(-gv[u]))));
    a.y[(long long)t * a.ldy + h * DH + lane + 64 * u] = f32_to_bf16_bits(y);
  }
}

// Key ranges: a workgroup covers NW·cw blocks of 64 of the pos cached keys (the last one also the t new tokens), cw
// chosen for about 1024 waves over the cache — one workgroup per CU, each wave streaming its chunks with one in
// flight.
struct Plan { int n_groups, group_len; };
// Waves per decode workgroup: 8 at head dim 128 with one row tile when the 4-wave plan would give each wave two or
// more chunks (32K: one chunk each, two waves per SIMD, the same key ranges and partials): 32K M = 1 22.5 → 20.0 µs.
// Where 4 waves hold one chunk each (4K, 16K), 8 would only halve the workgroups (4K 16.4 → 17.2 µs). More row tiles
// spill at two waves per SIMD. MI_GQA_NW=4 pins 4 (comparisons).
int gqa_waves(int d, int rows, int pos, int kv) {
  const char* e = getenv("MI_GQA_NW");
  if (d != 128 || rows > 16 || (e && atoi(e) == 4)) return kNW;
  return (long long)pos * kv > 256LL * kNW * BLOCK ? 8 : kNW;     // the 4-wave plan: two chunks or more per wave
}
Plan plan(int pos, int kv, int rows, int nw) {
  (void)rows;
  const char* e = getenv("MI_GQA_WAVES");             // MI_GQA_WAVES: tuning override
  const long long waves_target = e ? std::max(64LL, atoll(e)) : 256LL * nw;
  const int cw = (int)std::max<long long>(1, ((long long)pos * kv + waves_target * BLOCK - 1) / (waves_target * BLOCK));
  const int len = nw * cw * BLOCK;
  return {std::max(1, (pos + len - 1) / len), len};
}

// The merge runs inside the decode launch (the KV head's last workgroup) where its share of partials fits one pass
// (merge_fits); otherwise the gqa_merge launch. MI_GQA_FMERGE=0 pins the launch (comparisons).
bool fused_merge(int n_groups, int rows, int nw, int d) {
  const char* e = getenv("MI_GQA_FMERGE");
  if (e && atoi(e) == 0) return false;
  (void)d;
  return merge_fits(n_groups, rows, nw);
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// the arrival counters first, at a fixed place: a workspace shared by calls of other shapes keeps them zero
constexpr int KVMAX = 64;
struct Layout { size_t cnt, qf, qsc, part_o, part_ml, total; };
Layout layout(int kv, int n_groups, int rows, int d) {
  Layout l{};
  l.cnt = 0;
  l.qf = align256(KVMAX * sizeof(uint32_t));
  l.qsc = l.qf + align256((size_t)kv * MAXROWS * d * sizeof(uint16_t));
  l.part_o = l.qsc + align256((size_t)kv * MAXROWS * sizeof(float));
  l.part_ml = l.part_o + align256((size_t)kv * n_groups * rows * d * sizeof(float));
  l.total = l.part_ml + align256((size_t)kv * n_groups * rows * 2 * sizeof(float));
  return l;
}

template <int DH, bool BF>
int launch(const GqaArgs& a0, int rows, int nw, hipStream_t s) {
  GqaArgs a = a0;
  const dim3 grid(a.n_groups, a.kv), block(64 * nw);
  const int rt = (rows + 15) / 16;
  // Row tiles over workgroups (one tile each, a key range's tiles on one XCD) at head dim 256 — more tiles'
  // accumulators would spill — and at 128 while the grid stays within one workgroup per CU (4K, M = 8: 192
  // workgroups, 25.4 → 15.1 µs); MI_GQA_SPLIT=0 keeps several row tiles per workgroup at head dim 128 (comparisons).
  const char* e = getenv("MI_GQA_SPLIT");
  const bool split = DH == 256 || (!(e && atoi(e) == 0) && nw == kNW && (long long)a.n_groups * a.kv * rt <= 256);
  // The query rows and the append in the decode workgroups while each prepares at most 16 rows and the grid is
  // one round of CUs; otherwise their own launch (MI_GQA_PREP=1 forces it: comparisons).
  const char* ep = getenv("MI_GQA_PREP");
  const long long wgs = (long long)a.n_groups * a.kv * (split ? rt : 1);
  const bool prep = (ep && atoi(ep) == 1) || (split ? 16 : rows) > 16 || wgs > 256;
  if (prep) {
    hipLaunchKernelGGL((gqa_prep<DH, BF>), dim3(a.heads + a.kv, a.t), dim3(64), 0, s, a);
    MI_TRY_HIP(hipGetLastError(), "gqa_prep launch");
  } else {
    a.qf = nullptr;
    a.qsc = nullptr;
  }
  const bool own = !prep;
  if (split && rt > 1) {
    GqaArgs b = a;
    b.xcd_tiles = rt;
    const dim3 g1((a.n_groups * a.kv + 7) / 8 * rt * 8);
    if (own) hipLaunchKernelGGL((gqa_decode<1, DH, BF, kNW, true>), g1, block, 0, s, b);
    else hipLaunchKernelGGL((gqa_decode<1, DH, BF, kNW, false>), g1, block, 0, s, b);
  } else if (DH == 256 || rt == 1) {
    bool launched = false;
    if constexpr (DH == 128) {   // 8 waves: head dim 128, one row tile (gqa_waves)
      if (nw == 8) {
        if (own) hipLaunchKernelGGL((gqa_decode<1, DH, BF, 8, true>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((gqa_decode<1, DH, BF, 8, false>), grid, block, 0, s, a);
        launched = true;
      }
    }
    if (!launched) {
      if (own) hipLaunchKernelGGL((gqa_decode<1, DH, BF, kNW, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((gqa_decode<1, DH, BF, kNW, false>), grid, block, 0, s, a);
    }
  } else if constexpr (DH == 128) {   // several row tiles per workgroup: always after gqa_prep (rows > 16)
    if (rt == 2) hipLaunchKernelGGL((gqa_decode<2, DH, BF, kNW, false>), grid, block, 0, s, a);
    else if (rt == 3) hipLaunchKernelGGL((gqa_decode<3, DH, BF, kNW, false>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gqa_decode<4, DH, BF, kNW, false>), grid, block, 0, s, a);
  }
  MI_TRY_HIP(hipGetLastError(), "gqa_decode launch");
  if (a.fmerge) return MI_OK;
  hipLaunchKernelGGL((gqa_merge<DH>), dim3(a.heads, a.t), dim3(64 * MW), 0, s, a);
  MI_TRY_HIP(hipGetLastError(), "gqa_merge launch");
  return MI_OK;
}

}  // namespace

// the position the key ranges are planned for: the descriptor's, or — with a device position — the largest one the
// cache allows
int plan_pos(const mi_gqa_desc* d) { return d->pos_dev ? std::max(0, d->ctx_max - d->t) : d->pos; }

extern "C" size_t mi_gqa_workspace_bytes(const mi_gqa_desc* d) {
  if (!d || d->t < 1 || d->kv_heads < 1 || d->heads % d->kv_heads || d->head_dim < 1 || d->head_dim > DMAX) return 0;
  const int rows = d->heads / d->kv_heads * d->t;
  return layout(d->kv_heads, plan(plan_pos(d), d->kv_heads, rows, gqa_waves(d->head_dim, rows, plan_pos(d), d->kv_heads)).n_groups, rows, d->head_dim).total;
}

extern "C" int mi_gqa_decode(const mi_gqa_desc* d, void* stream) {
  MI_REQUIRE(d, "mi_gqa_decode: null descriptor");
  MI_REQUIRE(d->head_dim == 128 || d->head_dim == 256, "mi_gqa_decode: head_dim %d (built for 128 and 256)",
             d->head_dim);
  MI_REQUIRE(d->kv_dtype == MI_KV_INT8 || d->kv_dtype == MI_KV_BF16, "mi_gqa_decode: kv_dtype %d", d->kv_dtype);
  const bool bf = d->kv_dtype == MI_KV_BF16;
  MI_REQUIRE(d->t >= 1 && d->t <= TMAX, "mi_gqa_decode: t=%d must be in 1..%d", d->t, TMAX);
  MI_REQUIRE(d->kv_heads > 0 && d->kv_heads <= KVMAX && d->heads % d->kv_heads == 0,
             "mi_gqa_decode: kv_heads must be in 1..%d and divide heads", KVMAX);
  const int rep = d->heads / d->kv_heads;
  const int rows = rep * d->t;
  MI_REQUIRE(rows <= 64, "mi_gqa_decode: rep·t = %d query rows per KV head exceeds 64", rows);
  MI_REQUIRE(d->rotary_dim >= 0 && d->rotary_dim <= d->head_dim && d->rotary_dim % 2 == 0,
             "mi_gqa_decode: bad rotary_dim");
  MI_REQUIRE(d->pos_dev || (d->pos >= 0 && d->pos + d->t <= d->ctx_max), "mi_gqa_decode: pos + t exceeds the cache (%d)",
             d->ctx_max);
  MI_REQUIRE(d->ctx_max % BLOCK == 0, "mi_gqa_decode: ctx_max must be a multiple of %d", BLOCK);
  MI_REQUIRE(d->proj && d->k_codes && d->v_codes && d->y, "mi_gqa_decode: null pointer");
  MI_REQUIRE(bf || (d->k_scales && d->v_scales), "mi_gqa_decode: the int8 cache needs k_scales and v_scales");
  MI_REQUIRE(d->rotary_dim == 0 || (d->rope_cos && d->rope_sin), "mi_gqa_decode: RoPE tables missing");
  MI_REQUIRE(!d->qk_norm || (d->q_norm && d->k_norm), "mi_gqa_decode: qk_norm needs q_norm and k_norm");
  MI_REQUIRE(((uintptr_t)d->k_codes & 15) == 0 && ((uintptr_t)d->v_codes & 15) == 0, "mi_gqa_decode: cache alignment");
  MI_REQUIRE(!d->gate_src || (d->gate && d->ld_gate >= d->heads * d->head_dim),
             "mi_gqa_decode: gate_src needs gate = 1 and ld_gate >= heads·head_dim");
  GqaArgs a{};
  a.t = d->t; a.heads = d->heads; a.kv = d->kv_heads; a.d = d->head_dim; a.rot = d->rotary_dim; a.pos = d->pos;
  a.ctx = d->ctx_max; a.gate = d->gate; a.qk_norm = d->qk_norm; a.rep = rep; a.rows = rows;
  const int nw = gqa_waves(d->head_dim, rows, plan_pos(d), d->kv_heads);
  const Plan pl = plan(plan_pos(d), d->kv_heads, rows, nw);
  a.pos_dev = d->pos_dev;
  a.done = d->done;
  a.n_groups = pl.n_groups;
  a.group_len = pl.group_len;
  a.fmerge = fused_merge(pl.n_groups, rows, nw, d->head_dim);
  a.proj = d->proj; a.ldp = d->ld_proj; a.gsrc = d->gate_src; a.ldg = d->ld_gate; a.cosb = d->rope_cos; a.sinb = d->rope_sin;
  a.q_norm = d->q_norm; a.k_norm = d->k_norm; a.eps = d->eps; a.scaling = d->scaling;
  a.kc = d->k_codes; a.vc = d->v_codes;
  a.ks = bf ? nullptr : d->k_scales;
  a.vs = bf ? nullptr : d->v_scales;
  a.y = d->y; a.ldy = d->ld_y;
  const size_t need = mi_gqa_workspace_bytes(d);
  void* ws = d->workspace;
  if (ws) {
    MI_REQUIRE(d->workspace_bytes >= need, "mi_gqa_decode: workspace %zu B < %zu B", d->workspace_bytes, need);
  } else if (int rc = mi_library_scratch(MI_SCRATCH_GQA, need, static_cast<hipStream_t>(stream), &ws)) {
    return rc;
  }
  const Layout L = layout(d->kv_heads, a.n_groups, rows, d->head_dim);
  char* wb = static_cast<char*>(ws);
  a.cnt = reinterpret_cast<uint32_t*>(wb + L.cnt);
  a.qf = reinterpret_cast<uint16_t*>(wb + L.qf);
  a.qsc = reinterpret_cast<float*>(wb + L.qsc);
  a.part_o = reinterpret_cast<float*>(wb + L.part_o);
  a.part_ml = reinterpret_cast<float*>(wb + L.part_ml);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->head_dim == 128) return bf ? launch<128, true>(a, rows, nw, s) : launch<128, false>(a, rows, nw, s);
  return bf ? launch<256, true>(a, rows, nw, s) : launch<256, false>(a, rows, nw, s);
}
