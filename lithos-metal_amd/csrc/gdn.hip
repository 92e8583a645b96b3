// Gated DeltaNet decode step for T tokens (ops/gdn.py `gdn_mixer` + `gdn_norm`; nn/gdn.py:64-93; the kernel form
// kernels/common/gdn_mixer.metal:272-589): causal conv1d + SiLU over q|k|v, L2-normalised q (/√dk) and k,
// β = bf16(σ(b)), g = −exp(A_log)·softplus(a + dt_bias), the delta-rule recurrence on the FP32 state
// S ← S·e^g; Δ = (v − Sᵀk)·β; S += k⊗Δ; o = Sᵀq, then the gated RMSNorm y = bf16(bf16(w·bf16(o·r))·silu(z)).
//
// MI355X design: the state columns of a head are independent through the whole step (the Σ over dk stays inside a
// column), so a workgroup takes one value head's 32-column slice (grid hv × 4: 192 workgroups, enough to spread the
// 6 MB state stream over the chip), state waves of SC columns each plus two waves that compute the conv while
// the state streams in. Lane (c = l%SC, rg = l/SC) of a state wave holds the R = 128·SC/64 rows
// S[R·rg .. R·rg+R][col] in R VGPRs for all T tokens; the Σ over dk is R FMAs in-lane plus a shuffle reduction over
// the 64/SC lanes of the column, so the sequential token loop never touches memory or a barrier. One token takes
// SC = 16 (two state waves, 32 rows per lane); several take SC = 8 (four state waves, 16 rows per lane), halving
// each wave's serial work per token. Each workgroup computes the conv,
// SiLU and L2 norms of its key head's q/k (256 channels, repeated per slice: cheap) and of its own 32 v channels.
// Conv state is read from one buffer and written to another (several value heads read the same key head's
// channels: the reference solves the same race with two slots by step parity, gdn_mixer.metal:25-37); the
// recurrent state may be updated in place (each workgroup owns its slice). The gated RMSNorm needs the head's
// whole output, so it is a second small kernel (gdn_gated_norm), or — with defer_norm — left to the consumer: the
// output projection's GEMV applies it while staging its input.
#include "mi_common.h"

namespace {

constexpr int DK = 128, DV = 128, CW = 4, TMAX = 16;
constexpr int SLICE = 32, NSLICE = DV / SLICE; // a workgroup: one value head's 32-column slice, in state waves of
constexpr int CONV_WAVES = 2;                  // SC columns each, and 2 waves that compute the conv meanwhile

// v(l) + v(l ^ 8) inside a row of 16 lanes (DPP row rotate by 8), the same value in both lanes
__device__ __forceinline__ float add_xor8(float v) { return v + dpp_f<0x128>(v); }

struct GdnArgs {
  int t, hk, hv;
  const uint16_t* proj; int ldp, z_off, q_off, k_off, v_off;
  const uint16_t* ab; int ldab, a_off, b_off;
  const uint16_t* conv_w;
  const float* neg_exp_a;
  const float* dt_bias;
  const float* norm_w;
  const uint16_t* conv_in;
  uint16_t* conv_out;
  const float* rec_in;
  float* rec_out;
  uint16_t* y; int ldy;
  float eps;
  int commit;               // the speculative commit pass: state only, no read-out
  const int32_t* t_dev;     // device-resident token count (<= t), or null
  const uint32_t* done;     // the step state's stop flag, or null: when set the step takes no token
  const uint32_t* step;     // the step state's step counter, or null: conv_in is then two slots chosen by parity
  long long conv_slot;      // elements per conv-state slot
  const uint16_t* pre;      // the convolved q|k|v [t][ld_pre] (the conv ran in the input projection), or null
  int ld_pre;
};

// tokens this launch takes: the device count (commit pass) or t, and none once the program has stopped — with
// T = 0 the kernel copies conv_in → conv_out and rec_in → rec_out unchanged and writes no read-out
__device__ __forceinline__ int tokens_now(const GdnArgs& a) {
  if (a.done && *a.done) return 0;
  return a.t_dev ? min(max(*a.t_dev, 0), a.t) : a.t;
}

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float bf(const uint16_t* p, long long i) { return bf16_bits_to_f32(p[i]); }

// TT: a bound on the tokens (>= a.t), so the conv waves' loads are a fixed, unconditional set
// SC: columns per state wave — 16 (two state waves, 32 rows of the column per lane) or 8 (four state waves, 16 rows
// per lane: half the serial work per token, for launches of several tokens)
// PRE: the conv is done (the input projection's epilogue wrote the convolved q|k|v to a.pre): the conv waves read
// those values instead, and the conv state is not touched
template <int TT, int SC, bool PRE>
__global__ __launch_bounds__(64 * (SLICE / SC + CONV_WAVES)) void gdn_step(GdnArgs a) {
  constexpr int WAVES = SLICE / SC, RG = 64 / SC, R = DK / RG;
  __shared__ float qs[TMAX][DK];   // conv → silu → L2-norm (q also /√dk)
  __shared__ float ks[TMAX][DK];
  __shared__ float vs[TMAX][SLICE];
  __shared__ float beta_s[TMAX], eg_s[TMAX];
  const int h = blockIdx.x, sl = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the device words first (the oldest loads, so waiting for them waits for nothing else): the token count and
  // the step counter that picks the conv slots
  const int T = tokens_now(a);
  const uint32_t rd = a.step ? ((*a.step + (a.commit ? 1u : 0u)) & 1u) : 0u;
  const int rep = a.hv / a.hk;
  const int kh = h / rep;
  const int key_dim = a.hk * DK;

  // ---- waves 0..WAVES-1 load the state slice; the CONV_WAVES after them compute the conv meanwhile (the vector
  // memory counter is per wave, so the conv's loads do not queue behind the state's) ------------------------------
  const int c = lane % SC, rg = lane / SC;
  const int col = sl * SLICE + wave * SC + c;     // column in the head
  const int lcol = wave * SC + c;                 // column in the slice
  float s[R];
  if (wave < WAVES) {
    const float* sin = a.rec_in + (long long)h * DK * DV;
#pragma unroll
    for (int i = 0; i < R; ++i) s[i] = sin[(long long)(R * rg + i) * DV + col];
  } else {
    // ---- causal conv1d + SiLU over the head's q, k (key head kh) and this slice's v channels: CPT channels per
    // thread. Every load is issued before any is used and none is conditional (a channel index past the last
    // re-reads the last, rows past a.t - 1 re-read that row, and both conv slots are read when the step picks
    // one), so the whole section waits for one round of memory latency
    constexpr int NCH = 2 * DK + SLICE, CPT = (NCH + 64 * CONV_WAVES - 1) / (64 * CONV_WAVES);
    const int ct = tid - 64 * WAVES;
    const int tl = a.t - 1;
    const bool kw_writer = (h % rep) == 0 && sl == 0;   // the workgroup that writes its key head's q/k conv state
    const uint16_t* slot1 = a.step && !PRE ? a.conv_in + a.conv_slot : a.conv_in;
    int chs[CPT], offs[CPT];
    uint2 wv[CPT];
    uint16_t cs[2][CPT][CW - 1], xp[CPT][TT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int cidx = min(ct + 64 * CONV_WAVES * k, NCH - 1);
      const int i = cidx < DK ? cidx : cidx < 2 * DK ? cidx - DK : cidx - 2 * DK;
      chs[k] = cidx < DK ? kh * DK + i : cidx < 2 * DK ? key_dim + kh * DK + i : 2 * key_dim + h * DV + sl * SLICE + i;
      offs[k] = cidx < DK ? a.q_off + kh * DK + i : cidx < 2 * DK ? a.k_off + kh * DK + i : a.v_off + h * DV + sl * SLICE + i;
      if constexpr (PRE) {                        // the convolved values, in channel order
#pragma unroll
        for (int t = 0; t < TT; ++t) xp[k][t] = a.pre[(long long)min(t, tl) * a.ld_pre + chs[k]];
        continue;
      }
      wv[k] = *reinterpret_cast<const uint2*>(a.conv_w + (long long)chs[k] * CW);   // CW = 4 BF16 taps, 8 bytes
#pragma unroll
      for (int j = 0; j < CW - 1; ++j) {
        cs[0][k][j] = a.conv_in[(long long)chs[k] * (CW - 1) + j];
        cs[1][k][j] = slot1[(long long)chs[k] * (CW - 1) + j];
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) xp[k][t] = a.proj[(long long)min(t, tl) * a.ldp + offs[k]];
    }
    // gates per token: β = bf16(σ(b)), e^g with g = −exp(A_log)·softplus(a + dt_bias)
    const int tg = min(ct, tl);
    const uint16_t bq = a.ab[(long long)tg * a.ldab + a.b_off + h], aq = a.ab[(long long)tg * a.ldab + a.a_off + h];
    const float nea = a.neg_exp_a[h], dtb = a.dt_bias[h];

    uint16_t* conv_out = a.step ? const_cast<uint16_t*>(a.conv_in) + (rd ^ 1u) * a.conv_slot : a.conv_out;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int cidx = ct + 64 * CONV_WAVES * k;
      if (cidx >= NCH) break;
      const int i = cidx < DK ? cidx : cidx < 2 * DK ? cidx - DK : cidx - 2 * DK;
      float* dst = cidx < DK ? &qs[0][i] : cidx < 2 * DK ? &ks[0][i] : &vs[0][i];
      const int ld = cidx < 2 * DK ? DK : SLICE;
      if constexpr (PRE) {
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          if (t >= T) break;
          dst[t * ld] = bf16_bits_to_f32(xp[k][t]);
        }
        continue;
      }
      const bool writer = cidx < 2 * DK ? kw_writer : true;   // which workgroup writes this channel's conv state
      const float w[CW] = {bf16_bits_to_f32(wv[k].x & 0xFFFFu), bf16_bits_to_f32(wv[k].x >> 16),
                           bf16_bits_to_f32(wv[k].y & 0xFFFFu), bf16_bits_to_f32(wv[k].y >> 16)};
      float xs[CW - 1 + TT];
#pragma unroll
      for (int j = 0; j < CW - 1; ++j) xs[j] = bf16_bits_to_f32(rd ? cs[1][k][j] : cs[0][k][j]);
#pragma unroll
      for (int t = 0; t < TT; ++t) xs[CW - 1 + t] = t < T ? bf16_bits_to_f32(xp[k][t]) : 0.0f;
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= T) break;
        float y = 0.0f;
#pragma unroll
        for (int j = 0; j < CW; ++j) y = __fadd_rn(y, __fmul_rn(w[j], xs[j + t]));   // the oracle's y += w·x
        dst[t * ld] = round_bf16(silu_f(round_bf16(y)));
      }
      if (writer) {                 // the last CW-1 inputs of [state | x]
#pragma unroll
        for (int j = 0; j < CW - 1; ++j) {
          float v = xs[j];
#pragma unroll
          for (int t = 1; t <= TT; ++t) v = (t == T) ? xs[t + j] : v;
          conv_out[(long long)chs[k] * (CW - 1) + j] = f32_to_bf16_bits(v);
        }
      }
    }
    if (ct < T) {
      beta_s[ct] = round_bf16(sigmoid_f(bf16_bits_to_f32(bq)));
      eg_s[ct] = expf(nea * softplus_f(bf16_bits_to_f32(aq) + dtb));
    }
  }
  lds_barrier();        // LDS only: the state waves' loads stay in flight across it

  // ---- L2 norms: with at most CONV_WAVES tokens the conv waves take them (while the state streams in), otherwise
  // wave w takes tokens w, w + (waves), … ----------------------------------------------------------------------
  const bool few = T <= CONV_WAVES;
  for (int t = few ? wave - WAVES : wave; t >= 0 && t < T; t += few ? CONV_WAVES : WAVES + CONV_WAVES) {
    const float q0 = qs[t][lane], q1 = qs[t][lane + 64];
    const float k0 = ks[t][lane], k1 = ks[t][lane + 64];
    const float rq = 1.0f / sqrtf(wave_sum(q0 * q0 + q1 * q1) + 1e-6f);
    const float rk = 1.0f / sqrtf(wave_sum(k0 * k0 + k1 * k1) + 1e-6f);
    qs[t][lane] = (q0 * rq) / sqrtf((float)DK);
    qs[t][lane + 64] = (q1 * rq) / sqrtf((float)DK);
    ks[t][lane] = k0 * rk;
    ks[t][lane + 64] = k1 * rk;
  }
  lds_barrier();
  if (wave >= WAVES) return;

  // ---- the recurrence, token by token, state in registers. The token loop is unrolled over the bound TT and the
  // next token's k and q are read from LDS while this token computes, so the chain from one token to the next holds
  // no LDS latency; v, β and e^g of every token are read before the loop ------------------------------------------
  float vv[TT], bv[TT], ev[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) { vv[t] = vs[t][lcol]; bv[t] = beta_s[t]; ev[t] = eg_s[t]; }
  float kk[R], qq[R];
  auto stage = [&](int t, float* kd, float* qd) {
    const float4* k4 = reinterpret_cast<const float4*>(&ks[t][R * rg]);
    const float4* q4 = reinterpret_cast<const float4*>(&qs[t][R * rg]);
#pragma unroll
    for (int i = 0; i < R / 4; ++i) {
      const float4 kv = k4[i], qv = q4[i];
      kd[4 * i] = kv.x; kd[4 * i + 1] = kv.y; kd[4 * i + 2] = kv.z; kd[4 * i + 3] = kv.w;
      qd[4 * i] = qv.x; qd[4 * i + 1] = qv.y; qd[4 * i + 2] = qv.z; qd[4 * i + 3] = qv.w;
    }
  };
  stage(0, kk, qq);
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    if (t >= T) break;
    float kn[R], qn[R];
    if (t + 1 < TT) stage(t + 1, kn, qn);   // rows past T hold stale values and are never used
    const float e = ev[t];
    float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
#pragma unroll
    for (int i = 0; i < R; i += 4) {
      s[i] = __fmul_rn(s[i], e); s[i + 1] = __fmul_rn(s[i + 1], e);
      s[i + 2] = __fmul_rn(s[i + 2], e); s[i + 3] = __fmul_rn(s[i + 3], e);
      m0 = fmaf(s[i], kk[i], m0); m1 = fmaf(s[i + 1], kk[i + 1], m1);
      m2 = fmaf(s[i + 2], kk[i + 2], m2); m3 = fmaf(s[i + 3], kk[i + 3], m3);
    }
    float kv_part = (m0 + m1) + (m2 + m3);
    if (SC == 8) kv_part = add_xor8(kv_part);
    const float kv_mem = quad16_sum(kv_part);
    const float delta = (vv[t] - kv_mem) * bv[t];
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
    for (int i = 0; i < R; i += 4) {
      s[i] = __fadd_rn(s[i], __fmul_rn(kk[i], delta));
      s[i + 1] = __fadd_rn(s[i + 1], __fmul_rn(kk[i + 1], delta));
      s[i + 2] = __fadd_rn(s[i + 2], __fmul_rn(kk[i + 2], delta));
      s[i + 3] = __fadd_rn(s[i + 3], __fmul_rn(kk[i + 3], delta));
      o0 = fmaf(s[i], qq[i], o0); o1 = fmaf(s[i + 1], qq[i + 1], o1);
      o2 = fmaf(s[i + 2], qq[i + 2], o2); o3 = fmaf(s[i + 3], qq[i + 3], o3);
    }
    float o_part = (o0 + o1) + (o2 + o3);
    if (SC == 8) o_part = add_xor8(o_part);
    const float o = quad16_sum(o_part);
    if (rg == 0 && !a.commit) a.y[(long long)t * a.ldy + h * DV + col] = f32_to_bf16_bits(o);   // the BF16 read-out
    if (t + 1 < TT) {
#pragma unroll
      for (int i = 0; i < R; ++i) { kk[i] = kn[i]; qq[i] = qn[i]; }
    }
  }
  float* sout = a.rec_out + (long long)h * DK * DV;
#pragma unroll
  for (int i = 0; i < R; ++i) sout[(long long)(R * rg + i) * DV + col] = s[i];
}

// gated RMSNorm over each head's dv read-outs, in place: y = bf16(bf16(bf16(w)·bf16(o·r))·silu(z)); one wave per
// (head, token)
__global__ __launch_bounds__(64) void gdn_gated_norm(GdnArgs a) {
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  if (t >= tokens_now(a)) return;
  uint16_t* y = a.y + (long long)t * a.ldy + h * DV;
  const float v0 = bf16_bits_to_f32(y[lane]), v1 = bf16_bits_to_f32(y[lane + 64]);
  const float r = 1.0f / sqrtf(wave_sum(v0 * v0 + v1 * v1) / (float)DV + a.eps);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int cc = lane + 64 * j;
    const float n = round_bf16((j ? v1 : v0) * r);
    const float nw = round_bf16(round_bf16(a.norm_w[cc]) * n);
    const float z = bf(a.proj, (long long)t * a.ldp + a.z_off + h * DV + cc);
    y[cc] = f32_to_bf16_bits(nw * silu_f(z));
  }
}

}  // namespace

extern "C" int mi_gdn_step(const mi_gdn_desc* d, void* stream) {
  MI_REQUIRE(d, "mi_gdn_step: null descriptor");
  MI_REQUIRE(d->t >= 1 && d->t <= TMAX, "mi_gdn_step: t=%d must be in 1..%d", d->t, TMAX);
  MI_REQUIRE(d->dk == DK && d->dv == DV && d->conv_width == CW, "mi_gdn_step: built for dk=dv=%d, conv width %d", DK, CW);
  MI_REQUIRE(d->k_heads > 0 && d->v_heads > 0 && d->v_heads % d->k_heads == 0, "mi_gdn_step: v_heads must be a multiple of k_heads");
  MI_REQUIRE(d->proj && d->neg_exp_a && d->dt_bias && d->norm_w && d->rec_in && d->rec_out && (d->y || d->commit) &&
             (d->pre || (d->conv_w && d->conv_in && (d->conv_out || d->step))), "mi_gdn_step: null pointer");
  MI_REQUIRE(!d->pre || (!d->commit && d->t <= 2 && d->ld_pre >= 2 * d->k_heads * d->dk + d->v_heads * d->dv),
             "mi_gdn_step: pre (the projection's conv) is for a step of at most 2 tokens, not the commit pass, with "
             "ld_pre >= the conv channels");
  MI_REQUIRE(d->pre || (d->step ? !d->conv_out : d->conv_in != d->conv_out),
             "mi_gdn_step: conv_in and conv_out must be distinct buffers (shared key heads); with step, conv_in holds "
             "both slots and conv_out is NULL");
  // rec_in and rec_out may alias, in the commit pass too: each workgroup holds its state columns in registers from
  // the first load to the last store, and no other workgroup reads them
  GdnArgs a{};
  a.t = d->t; a.hk = d->k_heads; a.hv = d->v_heads;
  a.proj = d->proj; a.ldp = d->ld_proj; a.z_off = d->z_off; a.q_off = d->q_off; a.k_off = d->k_off; a.v_off = d->v_off;
  a.ab = d->ab ? d->ab : d->proj; a.ldab = d->ab ? d->ld_ab : d->ld_proj; a.a_off = d->a_off; a.b_off = d->b_off;
  a.conv_w = d->conv_w; a.neg_exp_a = d->neg_exp_a; a.dt_bias = d->dt_bias; a.norm_w = d->norm_w;
  a.conv_in = d->conv_in; a.conv_out = d->conv_out; a.rec_in = d->rec_in; a.rec_out = d->rec_out;
  a.y = d->y; a.ldy = d->ld_y; a.eps = d->eps;
  a.commit = d->commit; a.t_dev = d->t_dev; a.done = d->done;
  a.step = d->step;
  a.pre = d->pre; a.ld_pre = d->ld_pre;
  a.conv_slot = (long long)(2 * d->k_heads * d->dk + d->v_heads * d->dv) * (d->conv_width - 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // several tokens: four state waves of 8 columns (MI_GDN_SC=16 keeps two of 16)
  static const bool narrow_ok = [] { const char* e = getenv("MI_GDN_SC"); return !(e && atoi(e) == 16); }();
  const dim3 grid(d->v_heads, NSLICE), b16(64 * (SLICE / 16 + CONV_WAVES)), b8(64 * (SLICE / 8 + CONV_WAVES));
  if (d->pre) {                                 // the conv done by the projection (t <= 2)
    if (d->t == 1) hipLaunchKernelGGL((gdn_step<1, 16, true>), grid, b16, 0, s, a);
    else hipLaunchKernelGGL((gdn_step<2, 16, true>), grid, b16, 0, s, a);
  } else if (d->t == 1) hipLaunchKernelGGL((gdn_step<1, 16, false>), grid, b16, 0, s, a);
  else if (d->t <= 2) hipLaunchKernelGGL((gdn_step<2, 16, false>), grid, b16, 0, s, a);
  else if (!narrow_ok) {
    if (d->t <= 4) hipLaunchKernelGGL((gdn_step<4, 16, false>), grid, b16, 0, s, a);
    else if (d->t <= 8) hipLaunchKernelGGL((gdn_step<8, 16, false>), grid, b16, 0, s, a);
    else hipLaunchKernelGGL((gdn_step<TMAX, 16, false>), grid, b16, 0, s, a);
  } else if (d->t <= 4) hipLaunchKernelGGL((gdn_step<4, 8, false>), grid, b8, 0, s, a);
  else if (d->t <= 8) hipLaunchKernelGGL((gdn_step<8, 8, false>), grid, b8, 0, s, a);
  else hipLaunchKernelGGL((gdn_step<TMAX, 8, false>), grid, b8, 0, s, a);
  MI_TRY_HIP(hipGetLastError(), "gdn_step launch");
  if (!d->defer_norm && !d->commit) {
    hipLaunchKernelGGL(gdn_gated_norm, dim3(d->v_heads, d->t), dim3(64), 0, s, a);
    MI_TRY_HIP(hipGetLastError(), "gdn_gated_norm launch");
  }
  return MI_OK;
}
