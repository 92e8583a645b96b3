// The serial ops of a GPU-resident decode loop (ops/embed.py `embed`, ops/sample.py `argmax`, the advance of
// runtime/src/metal_core.mm:256-386 with the StepState fields of core/step_state.py:28-73): small kernels that run
// once per step so a captured step replays unchanged; everything that varies lives in mi_step_state.
#include "mi_common.h"

#include <time.h>

#include <chrono>
#include <deque>
#include <mutex>
#include <vector>

static_assert(sizeof(mi_step_state) == 272, "mi_step_state: the 272-byte layout");

namespace {

constexpr int EMBED_THREADS = 256;
constexpr int ARGMAX_THREADS = 256;

// one block per (token, 2048-column span): 8 BF16 per thread, 16-byte loads
__global__ __launch_bounds__(EMBED_THREADS) void embed_rows(mi_embed_desc d) {
  const int i = blockIdx.y;
  const int col = (blockIdx.x * EMBED_THREADS + threadIdx.x) * 8;
  if (col >= d.hidden) return;
  const int tok = d.tokens[i];
  const long long row = (tok >= 0 && tok < d.vocab) ? tok : 0;
  // T16 BF16 slab: tile = 16 rows × (hidden / 32) chunks of 512 elements; inside a chunk, column group q (8 columns)
  // of row r sits at q·128 + r·8
  const long long at = d.t16 ? ((row >> 4) * (d.hidden >> 5) + (col >> 5)) * 512 + ((col >> 3) & 3) * 128 + (row & 15) * 8
                             : row * d.hidden + col;
  const uint4 v = *reinterpret_cast<const uint4*>(d.table + at);
  *reinterpret_cast<uint4*>(d.out + (long long)i * d.ldo + col) = v;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);          // NaN compares false: never replaces a number
}

// The order "larger value, then lower index" over the numbers is total, so combining partial results in any order
// gives the same answer: the spans of a row run in parallel and the last one to finish folds them.
constexpr int ARGMAX_SPAN = ARGMAX_THREADS * 16;   // logits per workgroup
constexpr int ARGMAX_MAX_SPANS = 256;
constexpr size_t ARGMAX_COUNTERS = 256;            // bytes: 16 per-row arrival counters, padded

struct ArgmaxPartial { float v; int i; };

__device__ __forceinline__ void block_best(float& bv, int& bi, float* sv, int* si) {
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  bv = sv[0];
  bi = si[0];
  for (int k = 1; k < ARGMAX_THREADS / 64; ++k)
    if (better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
}

// ---- stochastic sampling (kernels/common/sample.metal, nn/sampling_ref.py) -------------------------------------
// The draw is argmax over the kept logits (v >= tau) of v / temperature + g_i, g_i = −log(−log(u_i)), u_i from a
// splitmix64 hash of (seed, step, token row, index): the reference's counter-based noise, so a draw is reproducible
// bit for bit and checkable against the host restatement.
struct SampleCtx {
  const float* tau;                // per row: the logit threshold (select_thresholds)
  float inv_t;
  uint32_t seed_lo, seed_hi, step;
  const mi_step_state* st;         // when set: seed = (rng_hi, rng_lo) and step come from the step state
};

__device__ __forceinline__ float uniform01(uint32_t seed_lo, uint32_t seed_hi, uint32_t step, uint32_t t, uint32_t i) {
  uint64_t x = ((uint64_t)seed_hi << 32) | seed_lo;
  x += (uint64_t)step * 0x9E3779B97F4A7C15ull + (uint64_t)t * 0xC2B2AE3D27D4EB4Full + (uint64_t)i * 0x165667B19E3779F9ull;
  x ^= x >> 30;                    // the splitmix64 finalizer
  x *= 0xBF58476D1CE4E5B9ull;
  x ^= x >> 27;
  x *= 0x94D049BB133111EBull;
  x ^= x >> 31;
  return ((float)((x >> 41) & 0x7FFFFFull) + 0.5f) * (1.0f / 8388608.0f);   // 23 bits: u in (0, 1), never 1
}

// BF16 bits → a 16-bit key that orders like the value (sign flipped: negative values reversed)
__device__ __forceinline__ uint32_t key16(uint32_t bits) { return bits & 0x8000u ? (~bits) & 0xFFFFu : bits | 0x8000u; }
__device__ __forceinline__ float key_val(uint32_t key) {
  const uint32_t bits = key & 0x8000u ? key & 0x7FFFu : (~key) & 0xFFFFu;
  return __uint_as_float(bits << 16);
}

constexpr uint32_t HIST_KEYS = 65536;
constexpr int SELECT_THREADS = 1024;
constexpr int SELECT_WAVES = SELECT_THREADS / 64;
constexpr uint32_t WAVE_KEYS = HIST_KEYS / SELECT_WAVES;   // keys per wave, descending from 65535 − 4096·w

// grid (spans, rows): the histogram of each row's logit keys (device-scope atomic adds; select clears it again)
__global__ __launch_bounds__(ARGMAX_THREADS) void sample_hist(const uint16_t* logits, int ld, int vocab, uint32_t* hist) {
  const int row = blockIdx.y;
  const uint16_t* p = logits + (long long)row * ld;
  uint32_t* h = hist + (size_t)row * HIST_KEYS;
  const int lo = blockIdx.x * ARGMAX_SPAN, hi = min(lo + ARGMAX_SPAN, vocab);
  for (int c = lo + (int)threadIdx.x; c < hi; c += ARGMAX_THREADS) atomicAdd(h + key16(p[c]), 1u);
}

// inclusive prefix over the 64 lanes of a wave (lane order)
template <typename T>
__device__ __forceinline__ T wave_scan_incl(T v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_total(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// the key where a descending cumulative sum starting at `run` first reaches `target`, walking this wave's keys
// (chunks of 64, lane 0 the highest key of a chunk); -inf when the wave's keys do not get there
template <bool MASS>
__device__ float walk_to(const uint32_t* h, uint32_t hi, float vmax, float inv_t, double run_in, double target, int lane) {
  float run = (float)run_in;
  float last = -INFINITY;                           // the lowest key with a count walked so far
  for (int q = 0; q < WAVE_KEYS / 64; ++q) {
    const uint32_t k = hi - 64 * q - lane;
    const uint32_t cnt = h[k];
    const float x = MASS ? (cnt ? (float)cnt * expf((key_val(k) - vmax) * inv_t) : 0.0f) : (float)cnt;
    const float incl = run + wave_scan_incl(x, lane);
    const unsigned long long hit = __ballot(cnt != 0u && incl >= (float)target);
    if (hit) return key_val(hi - 64 * q - (uint32_t)__builtin_ctzll(hit));
    const unsigned long long nz = __ballot(cnt != 0u);
    if (nz) last = key_val(hi - 64 * q - (63u - (uint32_t)__builtin_clzll(nz)));
    run = __shfl(incl, 63);
  }
  return last;                                      // the sums' order left the target a rounding short: the last key
}

// one workgroup per row (sample.metal `sample_select`): wave w owns the keys 65535 − 4096·w − [0, 4096), walked
// 64 at a time from the top (lane = key), so wave order is descending key order. tau = the most restrictive of
// top-k (the k-th largest logit, ties kept), top-p (the key at which the descending cumulative softmax mass of
// logits / temperature first reaches p of the total — of the top-k set's mass with flag 8) and min-p (max +
// temperature · log(min_p)). Per-wave sums (fixed lane order), then a sequential sum over the waves decides which
// wave walks to the key; the row's histogram is cleared after.
__global__ __launch_bounds__(SELECT_THREADS) void sample_select(uint32_t* hist, float* tau, int top_k, float temperature,
                                                                float top_p, float min_p, uint32_t flags) {
  __shared__ uint32_t wmax[SELECT_WAVES];
  __shared__ uint32_t wcnt[SELECT_WAVES];
  __shared__ float wmass[SELECT_WAVES], wmass_k[SELECT_WAVES];
  __shared__ float res[2];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, row = blockIdx.x;
  uint32_t* h = hist + (size_t)row * HIST_KEYS;
  const uint32_t hi = HIST_KEYS - 1 - (uint32_t)w * WAVE_KEYS;
  uint32_t km = 0;
  for (int q = 0; q < WAVE_KEYS / 64; ++q) {
    const uint32_t k = hi - 64 * q - lane;
    if (h[k]) km = max(km, k);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) km = max(km, (uint32_t)__shfl_xor((int)km, off));
  if (lane == 0) wmax[w] = km;
  if (threadIdx.x == 0) { res[0] = -INFINITY; res[1] = -INFINITY; }
  __syncthreads();
  uint32_t gmax = 0;
  for (int i = 0; i < SELECT_WAVES; ++i) gmax = max(gmax, wmax[i]);
  const float vmax = key_val(gmax), inv_t = 1.0f / temperature;
  float tau_k = -INFINITY, tau_p = -INFINITY, tau_m = -INFINITY;
  if (flags & 1u) {                                 // top-k: counts are exact
    uint32_t cnt = 0;
    for (int q = 0; q < WAVE_KEYS / 64; ++q) cnt += h[hi - 64 * q - lane];
    cnt = wave_total(cnt);
    if (lane == 0) wcnt[w] = cnt;
    __syncthreads();
    uint32_t before = 0;
    for (int i = 0; i < w; ++i) before += wcnt[i];
    if (before < (uint32_t)top_k && before + wcnt[w] >= (uint32_t)top_k) {
      const float kk = walk_to<false>(h, hi, vmax, inv_t, (double)before, (double)top_k, lane);
      if (lane == 0) res[0] = kk;
    }
    __syncthreads();
    tau_k = res[0];                                 // k beyond the vocabulary: every logit kept (−inf)
  }
  if (flags & 2u) {
    float m = 0.0f, mk = 0.0f;
    for (int q = 0; q < WAVE_KEYS / 64; ++q) {
      const uint32_t k = hi - 64 * q - lane;
      const uint32_t cnt = h[k];
      if (cnt) {
        const float x = (float)cnt * expf((key_val(k) - vmax) * inv_t);
        m += x;
        if (key_val(k) >= tau_k) mk += x;
      }
    }
    m = wave_total(m);
    mk = wave_total(mk);
    if (lane == 0) { wmass[w] = m; wmass_k[w] = mk; }
    __syncthreads();
    float total = 0.0f, before = 0.0f;
    for (int i = 0; i < SELECT_WAVES; ++i) total += (flags & 9u) == 9u ? wmass_k[i] : wmass[i];
    for (int i = 0; i < w; ++i) before += wmass[i];
    const float target = top_p * total;
    if (before < target && before + wmass[w] >= target) {
      const float kp = walk_to<true>(h, hi, vmax, inv_t, (double)before, (double)target, lane);
      if (lane == 0) res[1] = kp;
    }
    __syncthreads();
    tau_p = res[1];
  }
  if (flags & 4u) tau_m = vmax + temperature * logf(min_p);
  if (threadIdx.x == 0) tau[row] = fmaxf(fmaxf(tau_k, tau_p), tau_m);
  __syncthreads();                                  // every wave's reads before the clearing stores
  for (int q = 0; q < WAVE_KEYS / 64; ++q) {
    const uint32_t k = hi - 64 * q - lane;
    if (h[k]) h[k] = 0u;                            // clear for the next call
  }
}

// grid (spans, rows): each workgroup scans ARGMAX_SPAN logits of one row with 16-byte loads, publishes its best,
// and the last workgroup of the row to arrive folds the row's partials and resets the row's counter. SAMPLE: the
// value of a BF16 logit v >= tau is v / temperature + its Gumbel noise, any other logit is left out.
template <bool SAMPLE>
__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_spans(mi_argmax_desc d, uint32_t* counters,
                                                               ArgmaxPartial* part, SampleCtx sc) {
  __shared__ float sv[ARGMAX_THREADS / 64];
  __shared__ int si[ARGMAX_THREADS / 64];
  __shared__ int last;
  const int row = blockIdx.y, nb = gridDim.x, tid = threadIdx.x;
  const int lo = blockIdx.x * ARGMAX_SPAN, hi = min(lo + ARGMAX_SPAN, d.vocab);
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  float th = 0.0f;
  uint32_t seed_lo = 0, seed_hi = 0, step = 0;
  if constexpr (SAMPLE) {
    th = sc.tau[row];
    seed_lo = sc.st ? (uint32_t)sc.st->rng_lo : sc.seed_lo;
    seed_hi = sc.st ? (uint32_t)sc.st->rng_hi : sc.seed_hi;
    step = sc.st ? sc.st->step : sc.step;
  }
  if (!SAMPLE && d.f32) {
    const float* p = static_cast<const float*>(d.logits) + (long long)row * d.ld;
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | (uintptr_t)lo * 4) & 15) == 0;
    for (int c = lo + tid * 4; c < hi; c += ARGMAX_THREADS * 4) {
      float v[4];
      if (vec && c + 4 <= hi) {
        const float4 q = *reinterpret_cast<const float4*>(p + c);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
      } else {
        for (int e = 0; e < 4; ++e) v[e] = c + e < hi ? p[c + e] : NAN;
      }
      for (int e = 0; e < 4; ++e)
        if (better(v[e], c + e, bv, bi)) { bv = v[e]; bi = c + e; }
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(d.logits) + (long long)row * d.ld;
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | (uintptr_t)lo * 2) & 15) == 0;
    for (int c = lo + tid * 8; c < hi; c += ARGMAX_THREADS * 8) {
      uint32_t w[4];
      if (vec && c + 8 <= hi) {
        const uint4 q = *reinterpret_cast<const uint4*>(p + c);
        w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
      } else {
        for (int e = 0; e < 4; ++e) {
          const uint32_t a = c + 2 * e < hi ? p[c + 2 * e] : 0x7FC0u;          // past the end: NaN
          const uint32_t b = c + 2 * e + 1 < hi ? p[c + 2 * e + 1] : 0x7FC0u;
          w[e] = a | (b << 16);
        }
      }
      for (int e = 0; e < 4; ++e) {
        float v0 = __uint_as_float(w[e] << 16), v1 = __uint_as_float(w[e] & 0xFFFF0000u);
        if constexpr (SAMPLE) {
          v0 = v0 >= th ? v0 * sc.inv_t - logf(-logf(uniform01(seed_lo, seed_hi, step, row, c + 2 * e))) : NAN;
          v1 = v1 >= th ? v1 * sc.inv_t - logf(-logf(uniform01(seed_lo, seed_hi, step, row, c + 2 * e + 1))) : NAN;
        }
        if (better(v0, c + 2 * e, bv, bi)) { bv = v0; bi = c + 2 * e; }
        if (better(v1, c + 2 * e + 1, bv, bi)) { bv = v1; bi = c + 2 * e + 1; }
      }
    }
  }
  block_best(bv, bi, sv, si);
  if (tid == 0) {
    part[row * nb + blockIdx.x] = ArgmaxPartial{bv, bi};
    __threadfence();
    last = atomicAdd(&counters[row], 1u) == (uint32_t)(nb - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  bv = -INFINITY;
  bi = 0x7FFFFFFF;
  for (int k = tid; k < nb; k += ARGMAX_THREADS) {
    const ArgmaxPartial q = part[row * nb + k];
    if (better(q.v, q.i, bv, bi)) { bv = q.v; bi = q.i; }
  }
  __syncthreads();                                  // sv / si are reused
  block_best(bv, bi, sv, si);
  if (tid == 0) {
    d.ids[row] = bi == 0x7FFFFFFF ? -1 : bi;        // no number in the row
    atomicExch(&counters[row], 0u);
  }
}

__device__ __forceinline__ void publish_ctl(uint32_t* ctl, const mi_step_state* st) {
  if (ctl) {                                        // posted writes to pinned host memory: the pump polls these
    __atomic_store_n(&ctl[2], st->error, __ATOMIC_RELAXED);
    __atomic_store_n(&ctl[1], st->done, __ATOMIC_RELEASE);
  }
}

// one thread: the ring, the position and the stop conditions
__global__ __launch_bounds__(64) void advance_step(mi_advance_desc d) {
  if (threadIdx.x != 0) return;
  mi_step_state* st = d.state;
  if (st->done) return;
  const uint32_t t = min(max(st->t_this_step, 1u), (uint32_t)MI_STEP_T_MAX);   // a state the host left inconsistent
  if (st->prefill_left > 0) {                       // a prompt chunk: no token leaves the step
    st->position += t;
    st->step += 1;
    if (d.ctx_cap && st->position >= d.ctx_cap) { st->error = 2; st->done = 1; }
    publish_ctl(d.host_ctl, st);
    return;
  }
  const int32_t tok = d.tokens[t - 1];
  const uint32_t head = st->ring_head;
  if (head - st->ring_tail >= d.ring_cap) {         // the host has not drained: overflow
    st->error = 1;
    st->done = 1;
    publish_ctl(d.host_ctl, st);
    return;
  }
  d.ring[head % d.ring_cap] = ((uint64_t)(head + 1) << 32) | (uint32_t)tok;
  st->ring_head = head + 1;
  if (st->stop_at && head + 1 >= st->stop_at) st->done = 1;
  st->pending_tokens[0] = tok;
  st->position += t;
  st->step += 1;
  st->t_this_step = 1;
  for (int i = 0; i < d.n_eos; ++i)
    if (tok == d.eos[i]) st->done = 1;
  if (d.ctx_cap && st->position >= d.ctx_cap) { st->error = 2; st->done = 1; }
  publish_ctl(d.host_ctl, st);
}

int argmax_spans_of(int vocab) { return (vocab + ARGMAX_SPAN - 1) / ARGMAX_SPAN; }

__global__ void fill_neg_inf(float* p, int n) {
  if ((int)threadIdx.x < n) p[threadIdx.x] = -INFINITY;
}

__global__ __launch_bounds__(64) void verify_select_step(mi_verify_select_desc d) {
  if (threadIdx.x != 0) return;
  mi_step_state* st = d.state;
  if (st->done) return;
  if (d.lm) st->drafter_ctx_len = st->position + (st->prefill_left > 0 ? 0u : d.gamma);
  else st->drafter_ctx_len += st->n_inject;
  st->n_inject = 0;
  if (st->prefill_left > 0) return;                 // the host feeds the next prompt chunk
  for (uint32_t k = 0; k < d.gamma; ++k) {
    st->draft_tokens[k] = d.drafts[k];
    st->confidence[k] = d.conf[k];
    if (d.log_cap) d.conf_log[(st->step % d.log_cap) * 16 + k] = d.conf[k];
  }
  uint32_t lmax = min(d.gamma, d.t_max - 1);
  if (d.ctx_cap) {                                  // the verify rows position … position + L must fit the caches
    if (st->position >= d.ctx_cap) { st->error = 2; st->done = 1; return; }
    lmax = min(lmax, d.ctx_cap - st->position - 1);
  }
  uint32_t L = 0;
  if (d.mode == 2) {
    L = min((uint32_t)fmaxf(d.threshold, 0.f), lmax);
  } else if (d.mode == 1) {
    float survive = 1.f, expected = 1.f, best = 1.f / d.cost[0];
    for (uint32_t l = 1; l <= lmax; ++l) {
      survive *= d.conf[l - 1];
      expected += survive;
      const float score = expected / d.cost[l];
      if (score > best) { best = score; L = l; }
    }
  } else if (d.threshold <= 0.f) {
    L = lmax;
  } else {
    while (L < lmax && d.conf[L] >= d.threshold) ++L;
  }
  st->gamma = d.gamma;
  st->verify_len = L;
  st->pending_tokens[0] = st->anchor;
  for (uint32_t k = 0; k < L; ++k) st->pending_tokens[k + 1] = d.drafts[k];
  st->t_this_step = 1 + L;
}

__device__ __forceinline__ bool is_eos(const int32_t* eos, int n, int32_t tok) {
  bool hit = false;
  for (int i = 0; i < n; ++i) hit |= tok == eos[i];
  return hit;
}

__global__ __launch_bounds__(64) void accept_scan_step(mi_accept_scan_desc d) {
  if (threadIdx.x != 0) return;
  mi_step_state* st = d.state;
  if (st->done) return;
  // the step's rows and verify length as the state holds them, kept inside the token rows whatever the host left
  // there (t in 1..16, L <= t - 1), so no row index falls outside the step
  const uint32_t t = min(max(st->t_this_step, 1u), (uint32_t)MI_STEP_T_MAX);
  if (st->prefill_left > 0) {                       // a prompt chunk: nothing to verify; its rows are injected next
    if (d.log_cap) d.log[st->step % d.log_cap] = (t << 16) | 0xFFFFu;
    st->position += t;
    st->step += 1;
    st->n_inject = t;
    st->checkpoint_index = t;
    st->n_chain = 0;
    if (d.ctx_cap && st->position >= d.ctx_cap) { st->error = 2; st->done = 1; }
    publish_ctl(d.host_ctl, st);
    return;
  }
  const uint32_t L = min(st->verify_len, t - 1);
  const uint32_t base = t - 1 - L;                  // the anchor's row
  uint32_t acc = 0;
  while (acc < L && d.tokens[base + acc] == st->pending_tokens[base + acc + 1]) ++acc;
  const int32_t bonus = d.tokens[base + acc];
  uint32_t head = st->ring_head;
  if (head + acc + 1 - st->ring_tail > d.ring_cap) {  // not enough ring room: the host fell behind
    st->error = 1;
    st->done = 1;
    publish_ctl(d.host_ctl, st);
    return;
  }
  uint32_t committed = 0;
  int32_t last = bonus;
  bool stop = false;
  for (uint32_t k = 0; k <= acc; ++k) {
    const int32_t tok = k < acc ? st->pending_tokens[base + k + 1] : bonus;
    d.ring[head % d.ring_cap] = ((uint64_t)(head + 1) << 32) | (uint32_t)tok;
    ++head;
    ++committed;
    last = tok;
    if (is_eos(d.eos, d.n_eos, tok)) { stop = true; break; }   // nothing after the first EOS is committed
  }
  if (d.log_cap) d.log[st->step % d.log_cap] = (committed << 16) | (L << 8) | acc;
  st->ring_head = head;
  if (st->stop_at && head >= st->stop_at) stop = true;
  st->accepted = acc;
  st->anchor = last;
  st->position += base + committed;
  st->step += 1;
  st->verify_len = 0;
  st->t_this_step = 1;
  st->n_inject = base + committed;
  st->checkpoint_index = base + committed;
  st->n_chain = 1;
  if (d.lm) st->n_inject = st->position > st->drafter_ctx_len ? st->position - st->drafter_ctx_len : 0;
  if (stop) st->done = 1;
  if (d.ctx_cap && st->position >= d.ctx_cap) { st->error = 2; st->done = 1; }
  publish_ctl(d.host_ctl, st);
}

double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

double thread_cpu_ms() {
  timespec ts;
  clock_gettime(CLOCK_THREAD_CPUTIME_ID, &ts);
  return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

// take slots while the next expected sequence number is present (slots of batches still running may be written in
// any order, so the GPU's head is never trusted), then publish the tail
bool drain_ring(mi_runner_desc* d) {
  const volatile uint64_t* slots = d->ring;
  uint32_t tail = __atomic_load_n(&d->host_ctl[0], __ATOMIC_RELAXED);
  bool full = false;
  for (;;) {
    const uint64_t v = slots[tail % d->ring_capacity];
    if ((uint32_t)(v >> 32) != tail + 1) break;
    if (d->n_tokens >= d->tokens_capacity) { full = true; break; }
    d->tokens[d->n_tokens++] = (int32_t)(uint32_t)v;
    ++tail;
  }
  __atomic_store_n(&d->host_ctl[0], tail, __ATOMIC_RELEASE);
  return full;
}

}  // namespace

extern "C" {

int mi_runner_run(mi_runner_desc* d, mi_runner_stats* st) {
  MI_REQUIRE(d && st && d->graph_exec && (d->state || d->state_ring_tail) && d->ring && d->host_ctl &&
             (d->tokens || !d->tokens_capacity), "mi_runner_run: null pointer");
  MI_REQUIRE(!d->state_done == !d->state_error, "mi_runner_run: state_done and state_error go together");
  MI_REQUIRE(d->ring_capacity > 0 && d->launches_per_batch > 0 && d->in_flight > 0,
             "mi_runner_run: ring_capacity, launches_per_batch and in_flight must be >= 1");
  MI_REQUIRE(d->n_tokens <= d->tokens_capacity, "mi_runner_run: n_tokens exceeds tokens_capacity");
  *st = mi_runner_stats{};
  hipStream_t s = static_cast<hipStream_t>(d->stream);
  auto exec = static_cast<hipGraphExec_t>(d->graph_exec);
  struct Batch { hipEvent_t a, b; };
  std::vector<Batch> pool(d->in_flight);
  for (auto& b : pool) {
    MI_TRY_HIP(hipEventCreate(&b.a), "hipEventCreate");
    MI_TRY_HIP(hipEventCreate(&b.b), "hipEventCreate");
  }
  auto release = [&]() { for (auto& b : pool) { (void)hipEventDestroy(b.a); (void)hipEventDestroy(b.b); } };
  const double t0 = now_ms(), c0 = thread_cpu_ms();
  const uint64_t first = d->n_tokens;
  std::deque<size_t> pending;
  size_t next = 0;
  bool full = false;
  hipError_t err = hipSuccess;
  auto observe = [&]() {
    Batch& b = pool[pending.front()];
    pending.pop_front();
    const double w = now_ms();
    // poll with short sleeps: the pump thread stays idle while the GPU works (hipEventSynchronize spins)
    hipError_t e;
    while ((e = hipEventQuery(b.b)) == hipErrorNotReady) {
      const timespec nap{0, 20000};
      nanosleep(&nap, nullptr);
    }
    st->wait_ms += now_ms() - w;
    if (e != hipSuccess && err == hipSuccess) err = e;
    float ms = 0.f;
    if (e == hipSuccess && hipEventElapsedTime(&ms, b.a, b.b) == hipSuccess) st->gpu_ms += ms;
    st->batches++;
    full = drain_ring(d) || full;
    st->done = __atomic_load_n(d->state_done ? d->state_done : &d->host_ctl[1], __ATOMIC_ACQUIRE);
    st->error = __atomic_load_n(d->state_error ? d->state_error : &d->host_ctl[2], __ATOMIC_RELAXED);
  };
  while (st->launches < d->max_launches && !st->done && !full && err == hipSuccess &&
         (d->max_tokens == 0 || d->n_tokens - first < d->max_tokens)) {
    const double l = now_ms();
    const uint32_t n = (uint32_t)std::min<uint64_t>(d->launches_per_batch, d->max_launches - st->launches);
    Batch& b = pool[next];
    // the tail the GPU checks for overflow: the host's value when the copy runs (it only grows)
    if (d->state_ring_tail)       // a host-resident state: a newer tail than the copy would give is as correct
      __atomic_store_n(d->state_ring_tail, __atomic_load_n(&d->host_ctl[0], __ATOMIC_RELAXED), __ATOMIC_RELEASE);
    else
      err = hipMemcpyAsync(&d->state->ring_tail, &d->host_ctl[0], sizeof(uint32_t), hipMemcpyHostToDevice, s);
    if (err == hipSuccess) err = hipEventRecord(b.a, s);
    for (uint32_t i = 0; i < n && err == hipSuccess; ++i) err = hipGraphLaunch(exec, s);
    if (err == hipSuccess) err = hipEventRecord(b.b, s);
    st->launch_ms += now_ms() - l;
    if (err != hipSuccess) break;
    pending.push_back(next);
    next = (next + 1) % pool.size();
    st->launches += n;
    while (pending.size() >= d->in_flight) observe();
  }
  while (!pending.empty()) observe();
  st->wall_ms = now_ms() - t0;
  st->host_busy_ms = thread_cpu_ms() - c0;
  st->tokens = d->n_tokens - first;
  release();
  MI_TRY_HIP(err, "mi_runner_run");
  return MI_OK;
}

int mi_embed(const mi_embed_desc* d, void* stream) {
  MI_REQUIRE(d && d->tokens && d->table && d->out, "mi_embed: null pointer");
  MI_REQUIRE(d->t >= 1 && d->t <= 16 && d->vocab > 0 && d->hidden > 0 && d->hidden % 8 == 0 && d->ldo >= d->hidden &&
             d->ldo % 8 == 0, "mi_embed: bad shape");
  MI_REQUIRE(((uintptr_t)d->table & 15) == 0 && ((uintptr_t)d->out & 15) == 0, "mi_embed: table / out alignment");
  MI_REQUIRE(!d->t16 || d->hidden % 32 == 0, "mi_embed: a T16 table needs hidden %% 32 == 0");
  const dim3 grid((d->hidden / 8 + EMBED_THREADS - 1) / EMBED_THREADS, d->t);
  hipLaunchKernelGGL(embed_rows, grid, dim3(EMBED_THREADS), 0, static_cast<hipStream_t>(stream), *d);
  MI_TRY_HIP(hipGetLastError(), "embed launch");
  return MI_OK;
}

size_t mi_argmax_workspace_bytes(const mi_argmax_desc* d) {
  if (!d || d->t < 1 || d->vocab < 1) return 0;
  return ARGMAX_COUNTERS + (size_t)d->t * argmax_spans_of(d->vocab) * sizeof(ArgmaxPartial);
}

int mi_argmax(const mi_argmax_desc* d, void* stream) {
  MI_REQUIRE(d && d->logits && d->ids, "mi_argmax: null pointer");
  MI_REQUIRE(d->t >= 1 && d->t <= 16 && d->vocab > 0 && d->ld >= d->vocab, "mi_argmax: bad shape");
  const int nb = argmax_spans_of(d->vocab);
  MI_REQUIRE(nb <= ARGMAX_MAX_SPANS, "mi_argmax: vocab %d exceeds %d", d->vocab, ARGMAX_MAX_SPANS * ARGMAX_SPAN);
  const size_t need = mi_argmax_workspace_bytes(d);
  void* ws = d->workspace;
  if (ws) {
    MI_REQUIRE(d->workspace_bytes >= need, "mi_argmax: workspace %zu B < %zu B", d->workspace_bytes, need);
  } else if (int rc = mi_library_scratch(MI_SCRATCH_ARGMAX, need, static_cast<hipStream_t>(stream), &ws)) {
    return rc;
  }
  auto* counters = static_cast<uint32_t*>(ws);
  auto* part = reinterpret_cast<ArgmaxPartial*>(static_cast<char*>(ws) + ARGMAX_COUNTERS);
  hipLaunchKernelGGL(argmax_spans<false>, dim3(nb, d->t), dim3(ARGMAX_THREADS), 0, static_cast<hipStream_t>(stream),
                     *d, counters, part, SampleCtx{});
  MI_TRY_HIP(hipGetLastError(), "argmax launch");
  return MI_OK;
}

// workspace: argmax counters | partials | tau[16] | histograms [t][65536] u32
size_t sample_layout(int t, int vocab, size_t* off_tau, size_t* off_hist) {
  const size_t part = ARGMAX_COUNTERS + (size_t)t * argmax_spans_of(vocab) * sizeof(ArgmaxPartial);
  *off_tau = (part + 255) / 256 * 256;
  *off_hist = *off_tau + 256;
  return *off_hist + (size_t)t * HIST_KEYS * sizeof(uint32_t);
}

size_t mi_sample_workspace_bytes(const mi_sample_desc* d) {
  if (!d || d->t < 1 || d->vocab < 1) return 0;
  size_t a, b;
  return sample_layout(d->t, d->vocab, &a, &b);
}

int mi_sample(const mi_sample_desc* d, void* stream) {
  MI_REQUIRE(d && d->logits && d->ids, "mi_sample: null pointer");
  MI_REQUIRE(d->t >= 1 && d->t <= 16 && d->vocab > 0 && d->ld >= d->vocab, "mi_sample: bad shape");
  MI_REQUIRE(d->temperature > 0.0f && d->top_k >= 0 && d->top_p >= 0.0f && d->min_p >= 0.0f,
             "mi_sample: temperature > 0, top_k / top_p / min_p >= 0 (temperature 0 is mi_argmax)");
  const int nb = argmax_spans_of(d->vocab);
  MI_REQUIRE(nb <= ARGMAX_MAX_SPANS, "mi_sample: vocab %d exceeds %d", d->vocab, ARGMAX_MAX_SPANS * ARGMAX_SPAN);
  size_t off_tau, off_hist;
  const size_t need = sample_layout(d->t, d->vocab, &off_tau, &off_hist);
  void* ws = d->workspace;
  if (ws) {
    MI_REQUIRE(d->workspace_bytes >= need, "mi_sample: workspace %zu B < %zu B", d->workspace_bytes, need);
  } else if (int rc = mi_library_scratch(MI_SCRATCH_ARGMAX, need, static_cast<hipStream_t>(stream), &ws)) {
    return rc;
  }
  char* wb = static_cast<char*>(ws);
  auto* counters = reinterpret_cast<uint32_t*>(wb);
  auto* part = reinterpret_cast<ArgmaxPartial*>(wb + ARGMAX_COUNTERS);
  auto* tau = reinterpret_cast<float*>(wb + off_tau);
  auto* hist = reinterpret_cast<uint32_t*>(wb + off_hist);
  uint32_t flags = 0;
  if (d->top_k > 0) flags |= 1u;
  if (d->top_p > 0.0f && d->top_p < 1.0f) flags |= 2u;
  if (d->min_p > 0.0f) flags |= 4u;
  if (d->topp_in_topk) flags |= 8u;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (flags & 7u) {
    hipLaunchKernelGGL(sample_hist, dim3(nb, d->t), dim3(ARGMAX_THREADS), 0, s, d->logits, d->ld, d->vocab, hist);
    hipLaunchKernelGGL(sample_select, dim3(d->t), dim3(SELECT_THREADS), 0, s, hist, tau, d->top_k, d->temperature,
                       d->top_p, d->min_p, flags);
  } else {
    hipLaunchKernelGGL(fill_neg_inf, dim3(1), dim3(64), 0, s, tau, d->t);        // nothing to cut: keep every logit
  }
  mi_argmax_desc am{};
  am.t = d->t; am.vocab = d->vocab; am.logits = d->logits; am.ld = d->ld; am.f32 = 0; am.ids = d->ids;
  SampleCtx sc{tau, 1.0f / d->temperature, (uint32_t)d->seed, (uint32_t)(d->seed >> 32), d->step, d->state};
  hipLaunchKernelGGL(argmax_spans<true>, dim3(nb, d->t), dim3(ARGMAX_THREADS), 0, s, am, counters, part, sc);
  MI_TRY_HIP(hipGetLastError(), "sample launch");
  return MI_OK;
}

int mi_advance(const mi_advance_desc* d, void* stream) {
  MI_REQUIRE(d && d->state && d->tokens && d->ring, "mi_advance: null pointer");
  MI_REQUIRE(d->ring_cap >= 1 && d->n_eos >= 0 && d->n_eos <= 8, "mi_advance: ring_cap >= 1, n_eos in 0..8");
  hipLaunchKernelGGL(advance_step, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), *d);
  MI_TRY_HIP(hipGetLastError(), "advance launch");
  return MI_OK;
}

int mi_verify_select(const mi_verify_select_desc* d, void* stream) {
  MI_REQUIRE(d && d->state && (d->gamma == 0 || (d->drafts && d->conf)), "mi_verify_select: null pointer");
  MI_REQUIRE(d->gamma <= MI_STEP_GAMMA_MAX && d->t_max >= 1 && d->t_max <= MI_STEP_T_MAX && d->mode <= 2,
             "mi_verify_select: gamma <= %d, t_max in 1..%d, mode 0..2", MI_STEP_GAMMA_MAX, MI_STEP_T_MAX);
  MI_REQUIRE(!d->log_cap || d->conf_log, "mi_verify_select: log_cap without conf_log");
  if (d->mode == 1)
    for (uint32_t l = 0; l <= d->gamma && l < 16; ++l)
      MI_REQUIRE(d->cost[l] > 0.f, "mi_verify_select: cost[%u] must be positive", l);
  hipLaunchKernelGGL(verify_select_step, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), *d);
  MI_TRY_HIP(hipGetLastError(), "verify_select launch");
  return MI_OK;
}

int mi_accept_scan(const mi_accept_scan_desc* d, void* stream) {
  MI_REQUIRE(d && d->state && d->tokens && d->ring, "mi_accept_scan: null pointer");
  MI_REQUIRE(d->ring_cap >= 1 && d->n_eos >= 0 && d->n_eos <= 8, "mi_accept_scan: ring_cap >= 1, n_eos in 0..8");
  MI_REQUIRE(!d->log_cap || d->log, "mi_accept_scan: log_cap without log");
  hipLaunchKernelGGL(accept_scan_step, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), *d);
  MI_TRY_HIP(hipGetLastError(), "accept_scan launch");
  return MI_OK;
}

void* mi_host_alloc(size_t bytes) {
  void* p = nullptr;
  if (hipHostMalloc(&p, bytes, hipHostMallocCoherent) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return p;
}

int mi_host_free(void* p) {
  if (p) MI_TRY_HIP(hipHostFree(p), "hipHostFree");
  return MI_OK;
}

}  // extern "C"
