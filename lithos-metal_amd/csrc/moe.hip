// MoE router top-k + expert grouping, and the weighted combine (ops/moe.py `moe_route`, `moe_combine`;
// nn/moe.py:108-135; kernels/common/moe_route.metal:20-66, moe_combine.metal:19-49, moe_group.metal:8-47).
//
// Semantics: softmax in FP32 over the BF16 logits, k rounds of argmax over the probabilities with ties to the lowest
// expert index, the chosen probabilities optionally renormalized by their sum (taken in pick order), weights rounded
// to BF16 and stored as FP32. A round that finds no finite probability (a row of NaN logits) gives expert id -1 with
// weight 0, and that pair joins no expert group, so no expert GEMV ever reads past the expert table. Combine: Σ_j w_j·h_j (fused multiply-adds in slot order) (+ bf16(σ(gate))·shared)
// (+ residual) in FP32, one BF16 rounding.
//
// MI355X design:
//  * moe_route: one workgroup, one wave per token (T <= 16): each lane holds E/64 logits; max / sum / argmax are
//    DPP + permlane reductions. The same launch then turns the ids into expert groups for the grouped GEMV — one
//    record per distinct expert, in order of first use, holding the ≤ 16 (token, slot) pairs routed to it (pair
//    p = t·k + j, ascending) — so the expert GEMVs stream exactly the chosen experts, each once per step.
//  * moe_combine: one workgroup per token, 8 columns per lane with 16-byte loads.
#include "mi_common.h"
#include "route.h"

#include <algorithm>

namespace {

constexpr int MAX_PER_LANE = ROUTE_MAX_PER_LANE;   // E <= 512
constexpr int MAX_K = ROUTE_MAX_K;
constexpr int MAX_T = 16;
constexpr int GROUP_REC = 18;        // expert, count, 16 pair ids (the grouped GEMV's record)

struct RouteArgs {
  int t, n_experts, top_k, renorm, ld_logits, max_groups;
  const uint16_t* logits;
  int32_t* ids;
  float* weights;
  int32_t* groups;
  int shared_expert, shared_gate_col;           // shared_expert > 0: slot top_k of every token (the shared expert)
  int pairs_per_record;                         // 1..16: an expert's pairs in records of at most this many; 0: 16
};

__global__ __launch_bounds__(64 * MAX_T) void moe_route(RouteArgs a) {
  __shared__ int sel[MAX_T * (MAX_K + 1)];
  const int lane = threadIdx.x & 63, t = threadIdx.x >> 6;
  const int E = a.n_experts, k = a.top_k;
  const int ks = k + (a.shared_expert > 0 ? 1 : 0);   // slots per token (the shared expert last)
  if (t < a.t) {                                    // wave-uniform
    // the shared expert's gate logit first: its load is then in flight with the router row's
    const uint16_t gq = a.logits[(long long)t * a.ld_logits + max(a.shared_gate_col, 0)];
    int ce[MAX_K];
    float cw[MAX_K];
    route_topk(a.logits + (long long)t * a.ld_logits, E, k, a.renorm, lane, ce, cw);
    for (int r = 0; r < k; ++r) {
      if (lane == 0) {
        a.ids[t * ks + r] = ce[r];
        a.weights[t * ks + r] = cw[r];
      }
      sel[t * ks + r] = ce[r];
    }
    if (a.shared_expert > 0) {                      // the shared expert: weight bf16(σ(its gate's logit))
      if (lane == 0) {
        a.ids[t * ks + k] = a.shared_expert;
        a.weights[t * ks + k] = route_shared_weight(bf16_bits_to_f32(gq));
      }
      sel[t * ks + k] = a.shared_expert;
    }
  }
  if (!a.groups) return;                            // workgroup-uniform
  // groups: an expert's pairs, ascending, in records of at most PR pairs; the records of one expert consecutive, the
  // experts in order of first use. Per chosen expert, LDS holds its lowest pair and its pairs as a bit mask
  // (order-independent atomic min / or): a pair's rank is the popcount of its expert's bits below it, the count all
  // of them. The expert's first record is the scan, over the pairs in order, of the records each expert's first
  // pair opens (a wave scan, then the waves' totals) — no pass over the pairs.
  constexpr int PW = (MAX_T * (MAX_K + 1) + 31) / 32;     // words of a pair mask
  // indexed by expert id: the routed experts (< 512) and the shared expert (<= 512, checked on the host)
  __shared__ int first_use[64 * MAX_PER_LANE + 1];
  __shared__ uint32_t pmask[64 * MAX_PER_LANE + 1][PW];
  __shared__ int pre[64 * MAX_T];                   // the records opened before each pair
  __shared__ int wtot[MAX_T];
  const int PR = a.pairs_per_record > 0 ? a.pairs_per_record : GROUP_REC - 2;
  const int P = a.t * ks;
  const int p = threadIdx.x;
  __syncthreads();                                  // every wave's slots are in sel
  const int e = p < P ? sel[p] : -1;                // a pair without an expert (id -1) joins no group
  if (e >= 0) {                                     // clear the chosen experts' entries (idempotent)
    first_use[e] = P;
#pragma unroll
    for (int w = 0; w < PW; ++w) pmask[e][w] = 0u;
  }
  __syncthreads();
  if (e >= 0) {
    atomicMin(&first_use[e], p);
    atomicOr(&pmask[e][p >> 5], 1u << (p & 31));
  }
  __syncthreads();
  int first = p, rank = 0, count = 0;
  if (e >= 0) {
    first = first_use[e];
#pragma unroll
    for (int w = 0; w < PW; ++w) {
      const uint32_t m = pmask[e][w];
      count += __popc(m);
      rank += w < (p >> 5) ? __popc(m) : w == (p >> 5) ? __popc(m & ((1u << (p & 31)) - 1u)) : 0;
    }
  }
  const int opened = e >= 0 && first == p ? (count + PR - 1) / PR : 0;   // records an expert's first pair opens
  int inc = opened;                                 // inclusive scan over the wave's pairs
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(inc, off, 64);
    inc += lane >= off ? y : 0;
  }
  if (lane == 63) wtot[t] = inc;
  __syncthreads();
  int before = 0, total = 0;
  for (int w = 0; w < a.t; ++w) {
    before += w < t ? wtot[w] : 0;
    total += wtot[w];
  }
  pre[p] = before + inc - opened;
  __syncthreads();
  if (e >= 0) {
    const int q = rank / PR;
    int32_t* rec = a.groups + (long long)(pre[first] + q) * GROUP_REC;
    rec[2 + rank - q * PR] = p;
    if (rank == q * PR) { rec[0] = e; rec[1] = min(PR, count - q * PR); }
  }
  // the records past the last one: empty
  for (int r = total + p; r < a.max_groups; r += blockDim.x) {
    a.groups[(long long)r * GROUP_REC] = -1;
    a.groups[(long long)r * GROUP_REC + 1] = 0;
  }
}

struct CombineArgs {
  int t, hidden, top_k, ldh, ld_shared, ld_gate, ldr, ldo;
  const uint16_t* h;
  const float* weights;
  const uint16_t* shared;
  const uint16_t* shared_gate;
  const uint16_t* residual;
  uint16_t* out;
  const float* nn_w;        // the next RMSNorm of out (moe_combine<true>), or null
  uint16_t* nn_x;
  int ld_nn_x;
  float nn_eps;
};

__device__ __forceinline__ void bf16x8_to_f32(uint4 u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

// One 8-column vector of token t's output: Σ_j w·h (in slot order), the shared expert, the residual; one BF16
// rounding.
__device__ __forceinline__ uint4 combine_vec(const CombineArgs& a, int t, int c) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, x[8];
  for (int j = 0; j < a.top_k; ++j) {
    const float w = a.weights[t * a.top_k + j];
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(a.h + (long long)(t * a.top_k + j) * a.ldh + c), x);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(w, x[i], acc[i]);
  }
  if (a.shared) {
    const float g = 1.0f / (1.0f + expf(-bf16_bits_to_f32(a.shared_gate[(long long)t * a.ld_gate])));
    const float gb = round_bf16(g);
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(a.shared + (long long)t * a.ld_shared + c), x);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(gb, x[i], acc[i]);
  }
  if (a.residual) {
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(a.residual + (long long)t * a.ldr + c), x);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += x[i];
  }
  uint4 o;
  o.x = f32_to_bf16_bits(acc[0]) | ((uint32_t)f32_to_bf16_bits(acc[1]) << 16);
  o.y = f32_to_bf16_bits(acc[2]) | ((uint32_t)f32_to_bf16_bits(acc[3]) << 16);
  o.z = f32_to_bf16_bits(acc[4]) | ((uint32_t)f32_to_bf16_bits(acc[5]) << 16);
  o.w = f32_to_bf16_bits(acc[6]) | ((uint32_t)f32_to_bf16_bits(acc[7]) << 16);
  return o;
}

__global__ __launch_bounds__(256) void moe_combine(CombineArgs a) {
  const int t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= a.hidden) return;
  *reinterpret_cast<uint4*>(a.out + (long long)t * a.ldo + c) = combine_vec(a, t, c);
}

// The combine with the next RMSNorm of its output (the next layer's normalized input): one workgroup of 1024 per
// token, a thread per 8-column vector; the output goes to LDS, where the first 256 threads take Σ out² as
// norm_apply's threads do (vectors tid, tid + 256, … in order, fma, then the waves in order) — the same statistic,
// bit for bit — and every thread normalizes its vector: x = bf16((out·r)·w). hidden <= 8192.
constexpr int CN_NT = 1024;
constexpr int CN_SUM = 256;
__global__ __launch_bounds__(CN_NT) void moe_combine_norm(CombineArgs a) {
  __shared__ __attribute__((aligned(16))) uint4 ys[CN_NT];
  __shared__ float red[CN_SUM / 64];
  __shared__ float rsh;
  const int t = blockIdx.x, tid = threadIdx.x, nv = a.hidden / 8;
  const int c = 8 * min(tid, nv - 1);
  const float4 w0 = *reinterpret_cast<const float4*>(a.nn_w + c), w1 = *reinterpret_cast<const float4*>(a.nn_w + c + 4);
  const uint4 o = combine_vec(a, t, c);
  if (tid < nv) {
    *reinterpret_cast<uint4*>(a.out + (long long)t * a.ldo + 8 * tid) = o;
    ys[tid] = o;
  }
  lds_barrier();
  if (tid < CN_SUM) {
    float s = 0.0f;
    for (int jj = tid; jj < nv; jj += CN_SUM) {
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
    for (int w = 0; w < CN_SUM / 64; ++w) ssq += red[w];
    rsh = 1.0f / sqrtf(ssq / (float)a.hidden + a.nn_eps);
  }
  lds_barrier();
  const float r = rsh;
  const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
  const float w8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  uint32_t xo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = round_bf16((bf16_bits_to_f32(ow[i] & 0xFFFFu) * r) * w8[2 * i]);
    const float hi = round_bf16((bf16_bits_to_f32(ow[i] >> 16) * r) * w8[2 * i + 1]);
    xo[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
  }
  if (tid < nv) *reinterpret_cast<uint4*>(a.nn_x + (long long)t * a.ld_nn_x + 8 * tid) = uint4{xo[0], xo[1], xo[2], xo[3]};
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int mi_moe_route(const mi_moe_route_desc* d, void* stream) {
  MI_REQUIRE(d, "mi_moe_route: null descriptor");
  MI_REQUIRE(d->t >= 1 && d->t <= MAX_T, "mi_moe_route: t=%d must be in 1..%d", d->t, MAX_T);
  MI_REQUIRE(d->n_experts >= 1 && d->n_experts <= 64 * MAX_PER_LANE, "mi_moe_route: n_experts=%d must be in 1..%d",
             d->n_experts, 64 * MAX_PER_LANE);
  MI_REQUIRE(d->top_k >= 1 && d->top_k <= MAX_K && d->top_k <= d->n_experts, "mi_moe_route: top_k=%d out of range",
             d->top_k);
  MI_REQUIRE(d->logits && d->ids && d->weights && d->ld_logits >= d->n_experts, "mi_moe_route: bad logits / outputs");
  const int sh = d->shared_expert > 0 ? 1 : 0;
  MI_REQUIRE(!sh || (d->shared_expert >= d->n_experts && d->shared_expert <= 64 * MAX_PER_LANE &&
                     d->shared_gate_col >= 0 && d->shared_gate_col < d->ld_logits),
             "mi_moe_route: the shared expert's index must follow the routed experts (at most %d) and its gate column "
             "lie in the logits row", 64 * MAX_PER_LANE);
  MI_REQUIRE(d->pairs_per_record >= 0 && d->pairs_per_record <= GROUP_REC - 2,
             "mi_moe_route: pairs_per_record=%d must be in 0..%d", d->pairs_per_record, GROUP_REC - 2);
  MI_REQUIRE(!d->groups || d->max_groups >= (d->pairs_per_record > 0 ? d->t * (d->top_k + sh)
                                                                     : std::min(d->t * d->top_k, d->n_experts) + sh),
             "mi_moe_route: max_groups=%d cannot hold every record (t·slots with pairs_per_record, else the distinct "
             "experts)", d->max_groups);
  RouteArgs a{d->t, d->n_experts, d->top_k, d->renorm, d->ld_logits, d->max_groups, d->logits, d->ids, d->weights,
              d->groups, d->shared_expert, d->shared_gate_col, d->pairs_per_record};
  hipLaunchKernelGGL(moe_route, dim3(1), dim3(64 * d->t), 0, static_cast<hipStream_t>(stream), a);
  MI_TRY_HIP(hipGetLastError(), "moe_route launch");
  return MI_OK;
}

extern "C" int mi_moe_combine(const mi_moe_combine_desc* d, void* stream) {
  MI_REQUIRE(d, "mi_moe_combine: null descriptor");
  MI_REQUIRE(d->t >= 1 && d->top_k >= 1 && d->hidden >= 8 && d->hidden % 8 == 0,
             "mi_moe_combine: t, top_k >= 1 and hidden a multiple of 8 (t=%d k=%d hidden=%d)", d->t, d->top_k, d->hidden);
  MI_REQUIRE(d->h && d->weights && d->out, "mi_moe_combine: null pointer");
  MI_REQUIRE(!d->shared == !d->shared_gate, "mi_moe_combine: shared and shared_gate go together");
  MI_REQUIRE(d->ldh % 8 == 0 && d->ldo % 8 == 0 && (!d->shared || d->ld_shared % 8 == 0) &&
                 (!d->residual || d->ldr % 8 == 0),
             "mi_moe_combine: row strides must be multiples of 8");
  MI_REQUIRE(aligned16(d->h) && aligned16(d->out) && (!d->shared || aligned16(d->shared)) &&
                 (!d->residual || aligned16(d->residual)),
             "mi_moe_combine: 16-byte aligned rows");
  CombineArgs a{d->t, d->hidden, d->top_k, d->ldh, d->ld_shared, d->ld_gate, d->ldr, d->ldo,
                d->h, d->weights, d->shared, d->shared_gate, d->residual, d->out, nullptr, nullptr, 0, 0.0f};
  if (d->next_norm_w) {
    MI_REQUIRE(aligned16(d->next_norm_w) && d->next_x && aligned16(d->next_x) && d->ld_next_x >= d->hidden &&
                   d->ld_next_x % 8 == 0,
               "mi_moe_combine: the next norm needs a 16-byte aligned next_norm_w and next_x rows (ld >= hidden, "
               "multiple of 8)");
    if (d->hidden <= 8 * CN_NT) {               // one workgroup per token writes out and its norm
      a.nn_w = d->next_norm_w;
      a.nn_x = d->next_x;
      a.ld_nn_x = d->ld_next_x;
      a.nn_eps = d->next_eps;
      hipLaunchKernelGGL(moe_combine_norm, dim3(d->t), dim3(CN_NT), 0, static_cast<hipStream_t>(stream), a);
      MI_TRY_HIP(hipGetLastError(), "moe_combine_norm launch");
      return MI_OK;
    }
  }
  const dim3 grid((d->hidden / 8 + 255) / 256, d->t);
  hipLaunchKernelGGL(moe_combine, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  MI_TRY_HIP(hipGetLastError(), "moe_combine launch");
  if (d->next_norm_w) {                         // a wider row: the norm as its own launch (the same values)
    mi_norm_desc nd{};
    nd.t = d->t; nd.k = d->hidden; nd.h = d->out; nd.ldh = d->ldo; nd.stat = nullptr; nd.stat_parts = 1;
    nd.w = d->next_norm_w; nd.x = d->next_x; nd.ldx = d->ld_next_x; nd.eps = d->next_eps;
    return mi_norm_apply(&nd, stream);
  }
  return MI_OK;
}
