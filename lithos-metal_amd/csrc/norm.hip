// The decode layer's RMSNorm as standalone ops (ops/norm.py:11-12): rmsnorm_stat (stat[t] = Σ_k h[t][k]²,
// kernels/common/rmsnorm_stat.metal:18-40) and norm_apply (x = bf16(h·rsqrt(Σ stat / K + eps)·w), w the (1 + w)
// weight, norm_apply.metal:24-51) — for a lowered graph whose norm does not feed a GEMV directly (the GEMVs fuse it
// on load and never launch these).
//
// MI355X design: a workgroup of 256 threads per row, 16-byte loads and stores; each thread sums the squares of its
// vectors (strided by the workgroup), the four waves reduce with DPP / permlane and meet in LDS in wave order, so
// the statistic does not depend on scheduling. norm_apply with stat = NULL computes the statistic itself (one
// launch instead of two) in the same order as rmsnorm_stat.
#include "mi_common.h"

namespace {

constexpr int NT = 256;

struct NormArgs {
  int t, k, ldh, ldx, parts;
  const uint16_t* h;
  float* stat_out;          // rmsnorm_stat: [t][parts] (parts = 1 here)
  const float* stat_in;     // norm_apply: [t][parts] partial sums, or null
  const float* w;           // (1 + w) [k]
  uint16_t* x;
  float eps;
};

__device__ __forceinline__ float row_sumsq(const uint16_t* row, int k) {
  __shared__ float red[NT / 64];
  float s = 0.0f;
  for (int j = threadIdx.x; j < k / 8; j += NT) {
    const uint4 q = *reinterpret_cast<const uint4*>(row + 8 * j);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_bits_to_f32(v[i] & 0xFFFFu), hi = bf16_bits_to_f32(v[i] >> 16);
      s = fmaf(lo, lo, s);
      s = fmaf(hi, hi, s);
    }
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) t += red[w];
  return t;
}

__global__ __launch_bounds__(NT) void rmsnorm_stat(NormArgs a) {
  const int t = blockIdx.x;
  const float s = row_sumsq(a.h + (long long)t * a.ldh, a.k);
  if (threadIdx.x == 0) a.stat_out[t] = s;
}

__global__ __launch_bounds__(NT) void norm_apply(NormArgs a) {
  const int t = blockIdx.x;
  const uint16_t* row = a.h + (long long)t * a.ldh;
  float ssq;
  if (a.stat_in) {
    ssq = 0.0f;
    for (int i = 0; i < a.parts; ++i) ssq += a.stat_in[t * a.parts + i];
  } else {
    ssq = row_sumsq(row, a.k);
  }
  const float r = 1.0f / sqrtf(ssq / (float)a.k + a.eps);
  uint16_t* out = a.x + (long long)t * a.ldx;
  for (int j = threadIdx.x; j < a.k / 8; j += NT) {
    const uint4 q = *reinterpret_cast<const uint4*>(row + 8 * j);
    const float4 w0 = *reinterpret_cast<const float4*>(a.w + 8 * j);
    const float4 w1 = *reinterpret_cast<const float4*>(a.w + 8 * j + 4);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = round_bf16((bf16_bits_to_f32(v[i] & 0xFFFFu) * r) * wv[2 * i]);
      const float hi = round_bf16((bf16_bits_to_f32(v[i] >> 16) * r) * wv[2 * i + 1]);
      o[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
    }
    *reinterpret_cast<uint4*>(out + 8 * j) = uint4{o[0], o[1], o[2], o[3]};
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check(const mi_norm_desc* d, const char* name) {
  MI_REQUIRE(d, "%s: null descriptor", name);
  MI_REQUIRE(d->t >= 1 && d->t <= 4096, "%s: t=%d must be in 1..4096", name, d->t);
  MI_REQUIRE(d->k >= 8 && d->k % 8 == 0, "%s: k=%d must be a positive multiple of 8", name, d->k);
  MI_REQUIRE(d->h && al16(d->h) && d->ldh >= d->k && d->ldh % 8 == 0,
             "%s: h must be 16-byte aligned rows with a stride >= k, multiple of 8", name);
  return MI_OK;
}

}  // namespace

extern "C" int mi_rmsnorm_stat(const mi_norm_desc* d, void* stream) {
  if (int rc = check(d, "mi_rmsnorm_stat")) return rc;
  MI_REQUIRE(d->stat, "mi_rmsnorm_stat: null stat");
  NormArgs a{d->t, d->k, d->ldh, 0, 1, d->h, d->stat, nullptr, nullptr, nullptr, 0.0f};
  hipLaunchKernelGGL(rmsnorm_stat, dim3(d->t), dim3(NT), 0, static_cast<hipStream_t>(stream), a);
  MI_TRY_HIP(hipGetLastError(), "rmsnorm_stat launch");
  return MI_OK;
}

extern "C" int mi_norm_apply(const mi_norm_desc* d, void* stream) {
  if (int rc = check(d, "mi_norm_apply")) return rc;
  MI_REQUIRE(d->w && al16(d->w), "mi_norm_apply: w must be a 16-byte aligned float32 [k]");
  MI_REQUIRE(d->x && al16(d->x) && d->ldx >= d->k && d->ldx % 8 == 0, "mi_norm_apply: bad output x");
  MI_REQUIRE(!d->stat || d->stat_parts >= 1, "mi_norm_apply: stat_parts >= 1 with a stat");
  NormArgs a{d->t, d->k, d->ldh, d->ldx, d->stat_parts, d->h, nullptr, d->stat, d->w, d->x, d->eps};
  hipLaunchKernelGGL(norm_apply, dim3(d->t), dim3(NT), 0, static_cast<hipStream_t>(stream), a);
  MI_TRY_HIP(hipGetLastError(), "norm_apply launch");
  return MI_OK;
}
