// GQA decode attention over an int8 KV cache, T new tokens (ops/attention.py `gqa_decode` + `gqa_merge`;
// nn/attention.py:215-243; nn/oracle.py:112-134; kernels/common/gqa_decode.metal:32-302).
//
// Semantics: q|gate per head, k, v from the projection; optional q/k RMSNorm(1 + w); partial RoPE (rotate_half on
// the first rotary_dim dims, BF16 arithmetic, BF16 tables); the fresh k/v are quantized into the cache
// (per token and KV head: scale = f16(absmax / 127), code = rint(x / scale)); scores bf16(bf16(q·k)·D^-½) over the
// dequantized cache, causal inside the step; softmax in FP32 with P rounded to BF16; P·V in FP32 → BF16;
// × bf16(σ(gate)).
//
// MI355X design:
//  * Cache layout (this backend's): K codes [kv][ctx][D] int8, V codes transposed [kv][D][ctx] int8, scales
//    [kv][ctx] f16 — each operand an MFMA B tile read with 16- or 8-byte loads.
//  * gqa_decode: one wave per (KV head, split of the keys); the rep·T query rows of the KV head are A tiles of
//    v_mfma_f32_16x16x32_f16 (Q prescaled by a power of two into F16 range); int8 codes become exact F16 with
//    an XOR / byte-permute / packed subtract. QKᵀ and P·V run on MFMA, the softmax online per 64-key chunk; the
//    V scale folds into P (with a per-chunk power of two so it stays in F16 range). Each split writes
//    (O, m, l) partials. The split holding the new tokens also quantizes and appends them.
//  * gqa_merge: one wave per (head, token) folds the splits in order and applies the gate — deterministic.
#include "mi_common.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace {

constexpr int D = 128;
constexpr int CHUNK = 64;       // keys per inner step
constexpr int TMAX = 16;

struct GqaArgs {
  int t, heads, kv, rot, pos, ctx, gate, qk_norm, rep, rows, n_splits, split_len;
  const uint16_t* proj; int ldp;
  const uint16_t* cosb; const uint16_t* sinb;   // [ctx][rot] BF16
  const float* q_norm; const float* k_norm;     // (1 + w), [D]
  float eps, scaling;
  int8_t* kc; uint16_t* ks; int8_t* vc; uint16_t* vs;
  float* part_o; float* part_ml;                // [kv][split][rows][D], [kv][split][rows][2]
  uint16_t* y; int ldy;
};

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

// q/k head vector of token t after the optional (1+w) RMSNorm and partial RoPE, into dst[D] (BF16 values as f32).
// The whole wave cooperates: lane l handles dims l and l + 64.
__device__ void prep_vec(const GqaArgs& a, const uint16_t* src, const float* nw, int t, float* dst, int lane) {
  float x0 = bfv(src, lane), x1 = bfv(src, lane + 64);
  if (a.qk_norm) {
    const float ms = wave_sum(x0 * x0 + x1 * x1) / (float)D;
    const float r = 1.0f / sqrtf(ms + a.eps);
    x0 = round_bf16((x0 * r) * nw[lane]);
    x1 = round_bf16((x1 * r) * nw[lane + 64]);
  }
  dst[lane] = x0;
  dst[lane + 64] = x1;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int half = a.rot / 2;
  const int p = a.pos + t;
  float o[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = lane + 64 * u;
    const float xi = dst[i];
    if (i < a.rot) {
      const float c = bfv(a.cosb, (long long)p * a.rot + i), s = bfv(a.sinb, (long long)p * a.rot + i);
      const float rot = i < half ? -dst[i + half] : dst[i - half];
      o[u] = round_bf16(round_bf16(xi * c) + round_bf16(rot * s));
    } else {
      o[u] = xi;
    }
  }
  __builtin_amdgcn_wave_barrier();
  dst[lane] = o[0];
  dst[lane + 64] = o[1];
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// quantize a BF16-valued vector src[D] (LDS) into int8 codes + f16 scale (wave cooperative); returns nothing,
// writes codes to (dst_codes + stride · i) and the scale to *dst_scale
__device__ void quant_store(const float* src, int8_t* codes, long long stride, uint16_t* scale_out, int lane) {
  const float x0 = src[lane], x1 = src[lane + 64];
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const f16_t sh = (f16_t)(amax / 127.0f);
  const float sc = (float)sh;
  float c0 = 0.0f, c1 = 0.0f;
  if (sc > 0.0f) {
    c0 = fminf(fmaxf(rintf(x0 / sc), -127.0f), 127.0f);
    c1 = fminf(fmaxf(rintf(x1 / sc), -127.0f), 127.0f);
  }
  codes[stride * lane] = (int8_t)(int)c0;
  codes[stride * (lane + 64)] = (int8_t)(int)c1;
  if (lane == 0) *scale_out = __builtin_bit_cast(uint16_t, sh);
}

template <int RT>
__global__ __launch_bounds__(64) void gqa_decode(GqaArgs a) {
  // the KV head's query rows (BF16 values, row = t·rep + r) while the A tiles are built; then P'' of the chunk,
  // the P·V A-operand source
  __shared__ __attribute__((aligned(16))) float qbuf[RT * 16 * D];
  __shared__ float tmp[D];
  float (*qv)[D] = reinterpret_cast<float (*)[D]>(qbuf);
  f16_t (*pl)[CHUNK + 8] = reinterpret_cast<f16_t (*)[CHUNK + 8]>(qbuf);
  const int lane = threadIdx.x;
  const int j = blockIdx.y;                    // KV head
  const int sp = blockIdx.x;                   // split
  const int n_keys = a.pos + a.t;
  const int k_begin = sp * a.split_len;
  const bool last = sp == a.n_splits - 1;     // splits cut the cached keys; the last also takes the new tokens
  const int k_end = last ? n_keys : k_begin + a.split_len;
  const int q_cols = a.gate ? 2 * D : D;
  const int k_col0 = a.heads * q_cols + j * D;
  const int v_col0 = a.heads * q_cols + a.kv * D + j * D;

  // ---- the new tokens' k / v: quantized into the cache by the split that holds them ---------------------------
  if (last) {
    for (int t = 0; t < a.t; ++t) {
      const uint16_t* row = a.proj + (long long)t * a.ldp;
      const int p = a.pos + t;
      prep_vec(a, row + k_col0, a.k_norm, t, tmp, lane);
      quant_store(tmp, a.kc + ((long long)j * a.ctx + p) * D, 1, a.ks + (long long)j * a.ctx + p, lane);
      tmp[lane] = bfv(row + v_col0, lane);
      tmp[lane + 64] = bfv(row + v_col0, lane + 64);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      quant_store(tmp, a.vc + (long long)j * D * a.ctx + p, a.ctx, a.vs + (long long)j * a.ctx + p, lane);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    __threadfence_block();                     // the appended rows are read back below by this wave
  }

  // ---- the query rows: norm + RoPE, then per-row power-of-two prescale into F16 A tiles -----------------------
  for (int row = 0; row < a.rows; ++row) {
    const int t = row / a.rep, h = j * a.rep + (row - t * a.rep);
    prep_vec(a, a.proj + (long long)t * a.ldp + h * q_cols, a.q_norm, t, qv[row], lane);
  }
  for (int row = a.rows; row < RT * 16; ++row) { qv[row][lane] = 0.0f; qv[row][lane + 64] = 0.0f; }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int m16 = lane & 15, kg = lane >> 4;
  f16x8 qa[RT][4];
  float qscale[RT];                            // 2^p of this lane's A row (row = 16·rt + m16)
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float* qr = qv[rt * 16 + m16];
    float mx = 0.0f;
    for (int i = 0; i < D; ++i) mx = fmaxf(mx, fabsf(qr[i]));
    const int p = mx == 0.0f ? 0 : (int)((__float_as_uint(mx) >> 23) & 0xFF) - 127 - 14;
    const float inv = __uint_as_float((uint32_t)(127 - p) << 23);
    qscale[rt] = __uint_as_float((uint32_t)(127 + p) << 23);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) qa[rt][s][i] = (f16_t)(qr[32 * kg + 8 * s + i] * inv);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // qv reads done before pl (same LDS) is written
  __builtin_amdgcn_wave_barrier();

  // ---- online softmax over the split's keys, 64 per chunk ---------------------------------------------------
  f32x4 o[RT][8];
  float m_run[RT][4], l_run[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) o[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) { m_run[rt][i] = -INFINITY; l_run[rt][i] = 0.0f; }
  }
  int pv_cur = 0;                              // O is held in units of 2^pv_cur
  const int8_t* kbase = a.kc + (long long)j * a.ctx * D;
  const int8_t* vbase = a.vc + (long long)j * D * a.ctx;
  const uint16_t* ksb = a.ks + (long long)j * a.ctx;
  const uint16_t* vsb = a.vs + (long long)j * a.ctx;
  // the row of this lane's D element i (rows 4·kg + i of each row tile) and its token
  for (int k0 = k_begin; k0 < k_end; k0 += CHUNK) {
    // scores: S[row][key] for 4 key tiles of 16
    f32x4 sacc[RT][4];
    float kscale[4], vscale[4];
    bool kvalid[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int key = k0 + kt * 16 + m16;
      kvalid[kt] = key < k_end;
      const int kk = kvalid[kt] ? key : k_begin;
      const uint4 c0 = *reinterpret_cast<const uint4*>(kbase + (long long)kk * D + 32 * kg);
      const uint4 c1 = *reinterpret_cast<const uint4*>(kbase + (long long)kk * D + 32 * kg + 16);
      kscale[kt] = (float)__builtin_bit_cast(f16_t, ksb[kk]);
      vscale[kt] = kvalid[kt] ? (float)__builtin_bit_cast(f16_t, vsb[kk]) : 0.0f;
      const f16x8 b0 = i8x8_to_f16(c0.x, c0.y), b1 = i8x8_to_f16(c0.z, c0.w);
      const f16x8 b2 = i8x8_to_f16(c1.x, c1.y), b3 = i8x8_to_f16(c1.z, c1.w);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[rt][0], b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[rt][1], b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[rt][2], b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[rt][3], b3, acc, 0, 0, 0);
        sacc[rt][kt] = acc;
      }
    }
    // the chunk's V-scale prescale 2^-pv (keeps P'' = p·v_scale·2^-pv in F16 range)
    float vmax = fmaxf(fmaxf(vscale[0], vscale[1]), fmaxf(vscale[2], vscale[3]));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, off, 64));
    const int pv = vmax == 0.0f ? pv_cur : (int)((__float_as_uint(vmax) >> 23) & 0xFF) - 127 - 14;
    const float pv_inv = __uint_as_float((uint32_t)(127 - pv) << 23);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      // the row scales of this lane's D rows (4·kg + i): 2^p of the query row, via the A-row owner lanes
      float rs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) rs[i] = __shfl(qscale[rt], (lane & 48) | (4 * kg + i), 64);
      float mc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rt * 16 + 4 * kg + i;
        const int t = row / a.rep;
        const int qpos = a.pos + t;
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const int key = k0 + kt * 16 + m16;
          float sc = round_bf16(sacc[rt][kt][i] * rs[i] * kscale[kt]);
          sc = round_bf16(sc * a.scaling);
          const bool ok = kvalid[kt] && key <= qpos && row < a.rows;
          sacc[rt][kt][i] = ok ? sc : -INFINITY;
          mx = fmaxf(mx, sacc[rt][kt][i]);
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        mc[i] = mx;
      }
      float alpha[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mnew = fmaxf(m_run[rt][i], mc[i]);
        const float ex = (m_run[rt][i] == -INFINITY) ? 0.0f : __expf(m_run[rt][i] - mnew);
        alpha[i] = (mnew == -INFINITY) ? 1.0f : ex;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const float s = sacc[rt][kt][i];
          const float p = (s == -INFINITY) ? 0.0f : __expf(s - mnew);
          psum += p;
          const float pp = round_bf16(p) * vscale[kt] * pv_inv;
          pl[rt * 16 + 4 * kg + i][kt * 16 + m16] = (f16_t)pp;
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) psum += __shfl_xor(psum, off, 64);
        l_run[rt][i] = l_run[rt][i] * alpha[i] + psum;
        m_run[rt][i] = mnew;
      }
      const float resc = __uint_as_float((uint32_t)(127 + pv_cur - pv) << 23);   // 2^(pv_cur - pv)
#pragma unroll
      for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[rt][ct][i] *= alpha[i] * resc;
    }
    pv_cur = pv;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // O += P''·V
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f16x8 pa[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) pa[rt] = *reinterpret_cast<const f16x8*>(&pl[rt * 16 + m16][ks * 32 + 8 * kg]);
      const int key8 = k0 + ks * 32 + 8 * kg;
      const int keyc = key8 + 8 <= a.ctx ? key8 : 0;
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        const uint2 c = *reinterpret_cast<const uint2*>(vbase + (long long)(ct * 16 + m16) * a.ctx + keyc);
        const f16x8 bv = i8x8_to_f16(c.x, c.y);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) o[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt], bv, o[rt][ct], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- partials: O (in units of 2^pv_cur → scaled back), m, l -------------------------------------------------
  const float unscale = __uint_as_float((uint32_t)(127 + pv_cur) << 23);
  const long long base = ((long long)j * a.n_splits + sp) * a.rows;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = rt * 16 + 4 * kg + i;
      if (row >= a.rows) continue;
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) a.part_o[(base + row) * D + ct * 16 + m16] = o[rt][ct][i] * unscale;
      if (m16 == 0) {
        a.part_ml[(base + row) * 2] = m_run[rt][i];
        a.part_ml[(base + row) * 2 + 1] = l_run[rt][i];
      }
    }
}

// one wave per (query head, token): fold the splits in order, normalize, BF16, × bf16(σ(gate))
__global__ __launch_bounds__(64) void gqa_merge(GqaArgs a) {
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int j = h / a.rep;
  const int row = t * a.rep + (h - j * a.rep);
  float M = -INFINITY;
  for (int s = 0; s < a.n_splits; ++s) M = fmaxf(M, a.part_ml[(((long long)j * a.n_splits + s) * a.rows + row) * 2]);
  float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int s = 0; s < a.n_splits; ++s) {
    const long long b = ((long long)j * a.n_splits + s) * a.rows + row;
    const float m = a.part_ml[b * 2];
    if (m == -INFINITY) continue;
    const float w = __expf(m - M);
    l += w * a.part_ml[b * 2 + 1];
    o0 += w * a.part_o[b * D + lane];
    o1 += w * a.part_o[b * D + lane + 64];
  }
  float y0 = round_bf16(o0 / l), y1 = round_bf16(o1 / l);
  if (a.gate) {
    const uint16_t* g = a.proj + (long long)t * a.ldp + h * 2 * D + D;
    y0 = round_bf16(y0 * round_bf16(1.0f / (1.0f + __expf(-bfv(g, lane)))));
    y1 = round_bf16(y1 * round_bf16(1.0f / (1.0f + __expf(-bfv(g, lane + 64)))));
  }
  a.y[(long long)t * a.ldy + h * D + lane] = f32_to_bf16_bits(y0);
  a.y[(long long)t * a.ldy + h * D + lane + 64] = f32_to_bf16_bits(y1);
}

// splits of the pos cached keys, CHUNK-multiple lengths, about 512 waves in all; the last split also covers the
// t new tokens, so the wave that appends them is the only one that reads them
int plan_splits(int pos, int kv, int* split_len) {
  int len = ((pos * kv + 511) / 512 + CHUNK - 1) / CHUNK * CHUNK;
  len = std::max(len, CHUNK);
  *split_len = len;
  return std::max(1, (pos + len - 1) / len);
}

std::mutex g_mu;
std::vector<std::pair<void*, size_t>> g_ws;

int workspace(size_t bytes, void** out) {
  int dev = 0;
  MI_TRY_HIP(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1, {nullptr, 0});
  auto& w = g_ws[dev];
  if (w.second < bytes) {
    if (w.first) MI_TRY_HIP(hipFree(w.first), "hipFree(gqa workspace)");
    w = {nullptr, 0};
    MI_TRY_HIP(hipMalloc(&w.first, bytes), "hipMalloc(gqa workspace)");
    w.second = bytes;
  }
  *out = w.first;
  return MI_OK;
}

}  // namespace

extern "C" size_t mi_gqa_workspace_bytes(const mi_gqa_desc* d) {
  if (!d || d->t < 1 || d->kv_heads < 1 || d->heads % d->kv_heads) return 0;
  int len = 0;
  const int splits = plan_splits(d->pos, d->kv_heads, &len);
  const size_t rows = (size_t)(d->heads / d->kv_heads) * d->t;
  return (size_t)d->kv_heads * splits * rows * (D + 2) * sizeof(float);
}

extern "C" int mi_gqa_decode(const mi_gqa_desc* d, void* stream) {
  MI_REQUIRE(d, "mi_gqa_decode: null descriptor");
  MI_REQUIRE(d->head_dim == D, "mi_gqa_decode: built for head_dim %d", D);
  MI_REQUIRE(d->t >= 1 && d->t <= TMAX, "mi_gqa_decode: t=%d must be in 1..%d", d->t, TMAX);
  MI_REQUIRE(d->kv_heads > 0 && d->heads % d->kv_heads == 0, "mi_gqa_decode: heads must be a multiple of kv_heads");
  const int rep = d->heads / d->kv_heads;
  const int rows = rep * d->t;
  MI_REQUIRE(rows <= 64, "mi_gqa_decode: rep·t = %d query rows per KV head exceeds 64", rows);
  MI_REQUIRE(d->rotary_dim >= 0 && d->rotary_dim <= D && d->rotary_dim % 2 == 0, "mi_gqa_decode: bad rotary_dim");
  MI_REQUIRE(d->pos >= 0 && d->pos + d->t <= d->ctx_max, "mi_gqa_decode: pos + t exceeds the cache (%d)", d->ctx_max);
  MI_REQUIRE(d->ctx_max % 8 == 0, "mi_gqa_decode: ctx_max must be a multiple of 8");
  MI_REQUIRE(d->proj && d->k_codes && d->k_scales && d->v_codes && d->v_scales && d->y, "mi_gqa_decode: null pointer");
  MI_REQUIRE(d->rotary_dim == 0 || (d->rope_cos && d->rope_sin), "mi_gqa_decode: RoPE tables missing");
  MI_REQUIRE(!d->qk_norm || (d->q_norm && d->k_norm), "mi_gqa_decode: qk_norm needs q_norm and k_norm");
  MI_REQUIRE(((uintptr_t)d->k_codes & 15) == 0 && ((uintptr_t)d->v_codes & 7) == 0, "mi_gqa_decode: cache alignment");
  GqaArgs a{};
  a.t = d->t; a.heads = d->heads; a.kv = d->kv_heads; a.rot = d->rotary_dim; a.pos = d->pos; a.ctx = d->ctx_max;
  a.gate = d->gate; a.qk_norm = d->qk_norm; a.rep = rep; a.rows = rows;
  a.n_splits = plan_splits(d->pos, d->kv_heads, &a.split_len);
  a.proj = d->proj; a.ldp = d->ld_proj; a.cosb = d->rope_cos; a.sinb = d->rope_sin;
  a.q_norm = d->q_norm; a.k_norm = d->k_norm; a.eps = d->eps; a.scaling = d->scaling;
  a.kc = d->k_codes; a.ks = d->k_scales; a.vc = d->v_codes; a.vs = d->v_scales;
  a.y = d->y; a.ldy = d->ld_y;
  const size_t need = mi_gqa_workspace_bytes(d);
  void* ws = d->workspace;
  if (ws) {
    MI_REQUIRE(d->workspace_bytes >= need, "mi_gqa_decode: workspace %zu B < %zu B", d->workspace_bytes, need);
  } else if (int rc = workspace(need, &ws)) {
    return rc;
  }
  a.part_o = static_cast<float*>(ws);
  a.part_ml = a.part_o + (size_t)d->kv_heads * a.n_splits * rows * D;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(a.n_splits, d->kv_heads);
  const int rt = (rows + 15) / 16;
  if (rt == 1) hipLaunchKernelGGL(gqa_decode<1>, grid, dim3(64), 0, s, a);
  else if (rt == 2) hipLaunchKernelGGL(gqa_decode<2>, grid, dim3(64), 0, s, a);
  else if (rt == 3) hipLaunchKernelGGL(gqa_decode<3>, grid, dim3(64), 0, s, a);
  else hipLaunchKernelGGL(gqa_decode<4>, grid, dim3(64), 0, s, a);
  MI_TRY_HIP(hipGetLastError(), "gqa_decode launch");
  hipLaunchKernelGGL(gqa_merge, dim3(d->heads, d->t), dim3(64), 0, s, a);
  MI_TRY_HIP(hipGetLastError(), "gqa_merge launch");
  return MI_OK;
}
