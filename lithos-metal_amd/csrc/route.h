// The MoE router's top-k over one token's logits, for one wave (kernels/common/moe_route.metal:20-66; nn/moe.py:
// 383-393): softmax in FP32 over the BF16 logits, k rounds of argmax over the probabilities with ties to the lowest
// expert index, the chosen probabilities renormalized by their sum (taken in pick order) when renorm, weights
// rounded to BF16. A round that finds no finite probability (a row of NaN logits) gives expert -1, weight 0.
// Shared by moe_route and by the expert GEMV that routes for itself at one token, so both give the same ids and
// weights bit for bit.
#pragma once
#include "mi_common.h"

constexpr int ROUTE_MAX_PER_LANE = 8;   // E <= 512
constexpr int ROUTE_MAX_K = 16;

// NPL logits per lane (E <= 64·NPL); the whole wave calls it; every lane ends with the same ce[0..k) / cw[0..k)
template <int NPL>
__device__ __forceinline__ void route_topk_n(const uint16_t* logits, int E, int k, int renorm, int lane, int* ce,
                                             float* cw) {
  static_assert(NPL <= ROUTE_MAX_PER_LANE, "at most 512 experts");
  float v[NPL];
  uint16_t raw[NPL];
  // every load unconditional (an index past the experts re-reads the last logit, then masked), so they are all in
  // flight at once: a load whose value meets a branch is waited for there, one round trip each
#pragma unroll
  for (int i = 0; i < NPL; ++i) raw[i] = logits[min(lane + 64 * i, E - 1)];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? bf16_bits_to_f32(raw[i]) : -INFINITY;
    m = fmaxf(m, v[i]);
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? expf(v[i] - m) : 0.0f;
    s += v[i];
  }
  s = wave_sum(s);
#pragma unroll
  for (int i = 0; i < NPL; ++i) v[i] = lane + 64 * i < E ? v[i] / s : -1.0f;   // -1: absent or taken
  float wsum = 0.0f;
  for (int r = 0; r < k; ++r) {
    float best = -1.0f;
    int bi = 1 << 20;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (v[i] > best) { best = v[i]; bi = lane + 64 * i; }        // strictly greater: the lane's lowest index
    const float gmax = wave_max(best);
    const int e = (int)-wave_max(-(best == gmax ? (float)bi : (float)(1 << 20)));
    if (e >= E) {                     // no finite probability left (NaN logits): no expert, weight 0
      ce[r] = -1;
      cw[r] = 0.0f;
      continue;
    }
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (lane + 64 * i == e) v[i] = -1.0f;
    ce[r] = e;
    cw[r] = gmax;
    wsum += gmax;
  }
  for (int r = 0; r < k; ++r) cw[r] = round_bf16(renorm && wsum > 0.0f ? cw[r] / wsum : cw[r]);
}

// the wave's lanes hold 4 logits each up to 256 experts (the softmax and each pick's compares over half the
// registers), 8 up to 512; the same picks and weights bit for bit (a lane's absent logits add 0 to its sum)
__device__ __forceinline__ void route_topk(const uint16_t* logits, int E, int k, int renorm, int lane, int* ce,
                                           float* cw) {
  if (E <= 256) route_topk_n<4>(logits, E, k, renorm, lane, ce, cw);
  else route_topk_n<8>(logits, E, k, renorm, lane, ce, cw);
}

// the shared expert's weight: bf16(σ(its gate's logit))
__device__ __forceinline__ float route_shared_weight(float g) { return round_bf16(1.0f / (1.0f + expf(-g))); }
