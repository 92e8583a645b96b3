// A chain of dependent M = 1 NVFP4 GEMVs in one persistent launch — the fused projection tail of a decode layer
// (out_proj → gate|up → down, or gate|up → down): the MI355X counterpart of the reference's region / MLP fusion into
// one megakernel with bounded worker synchronization (compiler/region_fusion.py:25-58, compiler/mlp_fusion.py:103-130,
// the timeout check at runtime/engine.py:100-105). Each phase has the semantics of mi_gemv (ops/gemv.py:1-12;
// kernels/common/gemv_T.metal:232-587): y = x·Wᵀ with FP32 accumulation and one BF16 rounding, the input RMSNorm or
// the gated head norm fused on load, a residual or silu·mul epilogue, long K split with the splits added in order.
//
// Why one launch: every kernel boundary in a stream costs launch, ramp and a tail where part of the chip idles.
// Here one workgroup per CU walks the phases in order: it takes the work items of a phase strided by the grid
// (item = one 16-row tile × one K split, the gemv_row wave layout: wave w holds 4 chunks of the tile's K) with the
// weights of RING items in flight, loads the first items of the next phase, and only then waits until every item of
// the previous phase is done — so the weight stream of a phase starts while the last items of the one before it
// finish. Measured on one MI355X (27B MLP, M = 1, weights from HBM): 46–48 µs against 38–41 µs for the gate|up and
// down launches of gemv_row. A phase streams at ≈ 4.3 TB/s (two workgroups per CU run at very different paces, and
// dynamic item assignment through one device counter was slower still), and a phase boundary costs ≈ 5 µs (store
// acknowledgement, counter, then the next input's load) — more than the kernel boundary it replaces. So the layers
// use it only on request (MI_LAYER_CHAIN=1); it is kept, exact and tested, as the fused form to improve on.
//
// Memory ordering between workgroups (they sit on different XCDs, whose L2s are not coherent with each other),
// without fences (an agent-scope release writes back the whole L2): every value one phase hands to a later one —
// outputs, split partials — is written with device-scope stores or read-modify-writes (they reach the device's
// coherence point, past the XCD's L2) and read with device-scope loads (served from that point, never from a stale
// L2 line). A workgroup waits for its own stores to complete (s_waitcnt) before it adds its finished items to the
// phase's counter, and a waiting workgroup issues its loads of those values only after it has read the final count.
// The wait is bounded: past its spin limit a workgroup records an error in the control block and goes on, so a
// grid that cannot become resident together ends with wrong results and an error instead of hanging. The last
// workgroup to leave re-arms the counters for the next launch.
#include "mi_common.h"
#include "t16.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace {

constexpr int KW = 4;                  // chunks per wave
constexpr int S = 12;                  // waves per workgroup: a work item covers up to 48 chunks (6144 columns)
constexpr int MAX_PHASES = MI_CHAIN_MAX_PHASES;
constexpr int RING = 4;                // work items in flight per workgroup
constexpr uint32_t kSpinLimit = 1u << 22;   // ≈ 0.3 s of s_sleep(2) polls: far past any real wait

struct Phase {
  const uint8_t* w;
  const float* row_scale;
  const uint16_t* x;
  uint16_t* y;
  const uint16_t* res;
  const float* norm_w;
  const float* gnorm_w;
  const uint16_t* gnorm_z;
  float* part;                         // split partials [ks][n_tiles·16]
  uint32_t* fold_cnt;                  // per-tile arrival counters of the K splits
  long long tile_stride;
  float eps, gnorm_eps;
  int ld_gnorm_z;
  int n, k, chunks, n_tiles, ks, kc, epilogue, items;
  int x_chain, res_chain;              // produced earlier in this launch: device-scope loads
};

struct ChainArgs {
  Phase ph[MAX_PHASES];
  int n_phases;
  uint32_t* ctl;                       // [p] items finished in phase p, [MAX_PHASES] workgroups finished,
                                       // [MAX_PHASES + 1] error flag (sticky)
};

// ---- device-scope (coherent across XCDs) loads and stores --------------------------------------------------------
__device__ __forceinline__ uint4 ld16_dev(const void* p) {
  const auto* q = static_cast<const unsigned long long*>(p);
  const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return uint4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
}
__device__ __forceinline__ uint4 ld16(const void* p, bool dev) {
  return dev ? ld16_dev(p) : *static_cast<const uint4*>(p);
}
__device__ __forceinline__ float ld_bf16(const uint16_t* p, bool dev) {
  const uint16_t u = dev ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *p;
  return bf16_bits_to_f32(u);
}
__device__ __forceinline__ void st_bf16_dev(uint16_t* p, float v) {
  __hip_atomic_store(p, f32_to_bf16_bits(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// this wave's memory operations have completed (stores acknowledged by the coherence point)
__device__ __forceinline__ void wait_memory() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- one work item's weights in registers --------------------------------------------------------------------------
struct ItemWeights {
  uint4 q[KW];
  uint4 sv;
};

struct ItemGeom {
  int tile, split, c0, kw;
};

__device__ __forceinline__ ItemGeom geom(const Phase& P, int item, int wave) {
  ItemGeom g;
  g.tile = item % P.n_tiles;
  g.split = item / P.n_tiles;
  const int c0_raw = g.split * P.kc + wave * KW;
  g.kw = min(KW, min(P.chunks, (g.split + 1) * P.kc) - c0_raw);   // <= 0: this wave has no chunk in the item
  g.c0 = g.kw > 0 ? c0_raw : 0;
  return g;
}

__device__ __forceinline__ void load_weights(const Phase& P, const ItemGeom g, int lane, ItemWeights& w) {
  const uint8_t* tb = P.w + (long long)g.tile * P.tile_stride;
  const int gi = g.c0 >> 3;
  const uint8_t* sp = tb + nv_scale_off(gi, P.chunks);
  if (nv_piece(nv_group_chunks(gi, P.chunks)) == 16) {
    w.sv = *reinterpret_cast<const uint4*>(sp + 16 * lane);
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(sp + 8 * lane);
    w.sv = uint4{t.x, t.y, 0u, 0u};
  }
  const int kwl = max(g.kw, 1);
#pragma unroll
  for (int cc = 0; cc < KW; ++cc)
    w.q[cc] = *reinterpret_cast<const uint4*>(tb + nv_code_off(g.c0 + min(cc, kwl - 1)) + 16 * lane);
}

// LDS per workgroup: each wave's staged slices of the phase input, one per K split (a phase's items share them: a
// wave always covers the same chunks of its split), then per item parity the slice sums [S][16] (double-buffered:
// a wave may start the next item while wave 0 still reads this one's)
constexpr int MAX_KS = 3;
constexpr int XS_LD = KW * 128;
struct Smem {
  uint16_t xs[MAX_KS][S][XS_LD];
  float stat[S];
  float red[2][S][16];
};

// the chunk range of wave `wave` in K split `sp`
__device__ __forceinline__ void wave_range(const Phase& P, int sp, int wave, int& c0, int& kw) {
  const int c0_raw = sp * P.kc + wave * KW;
  kw = min(KW, min(P.chunks, (sp + 1) * P.kc) - c0_raw);
  c0 = kw > 0 ? c0_raw : 0;
}

// Stage this wave's slices of the phase input x (8 columns per lane and split), normalized when a norm is fused:
// the input RMSNorm's Σx² over the row from every wave's slice (one split), or the gated head norm per 128 columns.
__device__ __forceinline__ void stage_phase(const Phase& P, Smem& sm, int lane, int wave) {
  const bool xdev = P.x_chain;
  uint4 xv[MAX_KS];
  int per_row[MAX_KS], col0[MAX_KS];
#pragma unroll
  for (int sp = 0; sp < MAX_KS; ++sp) {
    int c0 = 0, kw = 0;
    if (sp < P.ks) wave_range(P, sp, wave, c0, kw);
    per_row[sp] = max(kw, 0) * 16;
    col0[sp] = c0 * 128 + min(lane, max(per_row[sp], 1) - 1) * 8;
    xv[sp] = sp < P.ks ? ld16(P.x + col0[sp], xdev) : uint4{0u, 0u, 0u, 0u};
  }
  if (P.norm_w) {                                    // ks == 1
    const float4 nv0 = *reinterpret_cast<const float4*>(P.norm_w + col0[0]);
    const float4 nv1 = *reinterpret_cast<const float4*>(P.norm_w + col0[0] + 4);
    float sq = 0.0f;
    if (lane < per_row[0]) {
      const uint32_t vv[4] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = bf16_bits_to_f32(vv[q] & 0xFFFFu), hi = bf16_bits_to_f32(vv[q] >> 16);
        sq = fmaf(lo, lo, fmaf(hi, hi, sq));
      }
    }
    sq = wave_sum(sq);
    if (lane == 0) sm.stat[wave] = sq;
    __syncthreads();
    float t = 0.0f;
    for (int ww = 0; ww < S; ++ww) t += sm.stat[ww];
    const float rr = 1.0f / sqrtf(t / (float)P.k + P.eps);
    const float wv[8] = {nv0.x, nv0.y, nv0.z, nv0.w, nv1.x, nv1.y, nv1.z, nv1.w};
    uint32_t vv[4] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = round_bf16((bf16_bits_to_f32(vv[q] & 0xFFFFu) * rr) * wv[2 * q]);
      const float hi = round_bf16((bf16_bits_to_f32(vv[q] >> 16) * rr) * wv[2 * q + 1]);
      vv[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
    }
    xv[0] = uint4{vv[0], vv[1], vv[2], vv[3]};
  } else if (P.gnorm_w) {                            // ks == 1
    const uint4 zv = *reinterpret_cast<const uint4*>(P.gnorm_z + col0[0]);
    const float4 nv0 = *reinterpret_cast<const float4*>(P.gnorm_w + (col0[0] & 127));
    const float4 nv1 = *reinterpret_cast<const float4*>(P.gnorm_w + (col0[0] & 127) + 4);
    uint32_t vv[4] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w};
    gated_head_norm8(vv, zv, nv0, nv1, P.gnorm_eps);
    xv[0] = uint4{vv[0], vv[1], vv[2], vv[3]};
  }
#pragma unroll
  for (int sp = 0; sp < MAX_KS; ++sp)
    if (lane < per_row[sp]) *reinterpret_cast<uint4*>(&sm.xs[sp][wave][lane * 8]) = xv[sp];
  wave_lds_sync();
}

// One work item from the staged input: the weights `w` were loaded before; as soon as the dot products have
// consumed them, the next item's weights (`next`, when it exists) are issued into the same registers, so they
// stream in while this item's slices meet and wave 0 finishes it.
__device__ __forceinline__ void run_item(const Phase& P, const ItemGeom g, ItemWeights& w, bool has_next,
                                         const ItemGeom next, Smem& sm, int parity, int lane, int wave) {
  const int gq = lane >> 4, m_row = lane & 15;
  const int row = g.tile * 16 + m_row;
  float rs = 1.0f, res = 0.0f;                       // wave 0's epilogue operands, requested up front
  if (wave == 0) {
    const int r = min(row, P.n - 1);
    if (P.row_scale) rs = P.row_scale[row];
    if (P.epilogue == MI_EPI_RESIDUAL) res = ld_bf16(P.res + r, P.res_chain);
  }
  const uint16_t* xs = sm.xs[g.split][wave];
  // ---- the slice's dot products (e2m1 × 2^E exact in BF16, the scale's mantissa once per block of 16) -----------
  float acc = 0.0f;
#pragma unroll
  for (int cc = 0; cc < KW; ++cc) {
    if (cc >= g.kw) break;
    const uint32_t dw[4] = {w.q[cc].x, w.q[cc].y, w.q[cc].z, w.q[cc].w};
    uint4 xq[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) xq[s] = *reinterpret_cast<const uint4*>(xs + cc * 128 + 32 * gq + 8 * s);
    const uint32_t word = (g.c0 & 4) ? (cc < 2 ? w.sv.z : w.sv.w) : (cc < 2 ? w.sv.x : w.sv.y);
    const f32x2 f = (cc & 1) ? __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true)
                             : __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
    const uint32_t u0 = __float_as_uint(f.x), u1 = __float_as_uint(f.y);
    const float e[2] = {__uint_as_float(u0 & 0x7F800000u), __uint_as_float(u1 & 0x7F800000u)};
    const float mant[2] = {nv_mant(u0), nv_mant(u1)};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float part = 0.0f;
#pragma unroll
      for (int s = 2 * b; s < 2 * b + 2; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t xw = j == 0 ? xq[s].x : j == 1 ? xq[s].y : j == 2 ? xq[s].z : xq[s].w;
          part = __builtin_amdgcn_fdot2_f32_bf16(cvt_fp4x2_bf16(dw[s], e[b], j), __builtin_bit_cast(bf16x2, xw), part,
                                                 false);
        }
      acc = fmaf(part, mant[b], acc);
    }
  }
  if (has_next) load_weights(P, next, lane, w);
  const float v = quad16_sum(acc);
  if (gq == 0) sm.red[parity][wave][m_row] = v;
  __syncthreads();
  if (wave != 0) return;

  // ---- wave 0: the K slices in order, the K splits (last arriving split adds them in split order), epilogue ------
  float vt = slice_sum(&sm.red[parity][0][0], 16, S, lane);
  if (P.ks > 1) {
    auto* pu = reinterpret_cast<uint32_t*>(P.part);
    const long long pstride = (long long)P.n_tiles * 16;
    uint32_t seen = 0;
    if (gq == 0)
      seen = __hip_atomic_exchange(pu + g.split * pstride + row, __float_as_uint(vt), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(seen) : "memory");        // the exchange has returned
    uint32_t prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(P.fold_cnt + g.tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != (uint32_t)(P.ks - 1)) return;
    float s = 0.0f;
    if (gq == 0)
      for (int sp = 0; sp < P.ks; ++sp)
        s += __uint_as_float(__hip_atomic_fetch_or(pu + sp * pstride + row, 0u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
    vt = s;
    if (lane == 0) __hip_atomic_store(P.fold_cnt + g.tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  vt *= rs;
  const float up = __shfl_down(vt, 8, 16);
  if (gq != 0) return;
  if (P.epilogue == MI_EPI_SILU_MUL || P.epilogue == MI_EPI_SILU_MUL_ROUNDED) {
    const int col = g.tile * 8 + m_row;
    if (m_row >= 8 || col >= P.n / 2) return;
    const float o = P.epilogue == MI_EPI_SILU_MUL_ROUNDED ? silu_f(round_bf16(vt)) * round_bf16(up) : silu_f(vt) * up;
    st_bf16_dev(P.y + col, o);
  } else {
    if (row >= P.n) return;
    st_bf16_dev(P.y + row, P.epilogue == MI_EPI_RESIDUAL ? vt + res : vt);
  }
}

// thread 0 polls the count with bounded sleeps; the workgroup leaves the barrier together
__device__ __forceinline__ void wait_for(uint32_t* ctl, int p, uint32_t target) {
  if (threadIdx.x == 0) {
    uint32_t spins = 0;
    while (__hip_atomic_load(ctl + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > kSpinLimit) {
        __hip_atomic_store(ctl + MAX_PHASES + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
  asm volatile("" ::: "memory");
}

__global__ __launch_bounds__(64 * S) void gemv_chain(ChainArgs a) {
  __shared__ __attribute__((aligned(16))) Smem sm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  int parity = 0;
#pragma unroll
  for (int p = 0; p < MAX_PHASES; ++p) {      // unrolled: a phase's fields are read at constant kernarg offsets
    if (p >= a.n_phases) break;
    const Phase& P = a.ph[p];
    // Work items strided by the grid (one workgroup per CU: two sharing a CU run at very different paces, which
    // left each phase to the slowest). RING items are in flight per workgroup: their weights sit in a register
    // ring, and a slot is refilled with the item RING positions ahead as soon as its dot products are done; the
    // first RING items of a phase stream in during the wait for the phase before it.
    ItemWeights w0, w1, w2, w3;
    ItemGeom g0{}, g1{}, g2{}, g3{};
    const int b0 = blockIdx.x;
    auto prefetch = [&](ItemWeights& w, ItemGeom& g, int item) {
      if (item < P.items) {
        g = geom(P, item, wave);
        load_weights(P, g, lane, w);
      }
    };
    prefetch(w0, g0, b0);
    prefetch(w1, g1, b0 + G);
    prefetch(w2, g2, b0 + 2 * G);
    prefetch(w3, g3, b0 + 3 * G);
    if (p > 0) wait_for(a.ctl, p - 1, (uint32_t)a.ph[p - 1].items);
    stage_phase(P, sm, lane, wave);
    int done = 0;
#define MI_CHAIN_SLOT(K, W, GG)                                                                              \
    {                                                                                                        \
      const int it = item + (K) * G, nx = it + RING * G;                                                     \
      if (it >= P.items) break;                                                                              \
      run_item(P, GG, W, nx < P.items, geom(P, nx, wave), sm, parity, lane, wave);                           \
      parity ^= 1;                                                                                           \
      ++done;                                                                                                \
      GG = geom(P, nx, wave);                                                                                \
    }
    for (int item = b0; item < P.items; item += RING * G) {
      MI_CHAIN_SLOT(0, w0, g0)
      MI_CHAIN_SLOT(1, w1, g1)
      MI_CHAIN_SLOT(2, w2, g2)
      MI_CHAIN_SLOT(3, w3, g3)
    }
#undef MI_CHAIN_SLOT
    // this workgroup's outputs of the phase have reached the coherence point before the count says so
    wait_memory();
    __syncthreads();
    if (threadIdx.x == 0 && done)
      __hip_atomic_fetch_add(a.ctl + p, (uint32_t)done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(a.ctl + MAX_PHASES, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)G - 1) {                   // everyone is past every wait: re-arm for the next launch
      for (int p = 0; p < MAX_PHASES; ++p) __hip_atomic_store(a.ctl + p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctl + MAX_PHASES, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

int cu_count_now() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    n = 256;
  (void)hipGetLastError();
  return std::max(n, 1);
}

int blocks_per_cu() {
  static int cached = 0;
  if (!cached) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(gemv_chain), 64 * S, 0) !=
            hipSuccess || n < 1)
      n = 1;
    (void)hipGetLastError();
    cached = std::min(n, 1);
  }
  return cached;
}

bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
  const char* pa = static_cast<const char*>(a);
  const char* pb = static_cast<const char*>(b);
  return pa < pb + bn && pb < pa + an;
}

// control block | per phase: fold counters (n_tiles) | partials (ks · n_tiles · 16 floats)
constexpr size_t kCtlBytes = 256;
size_t phase_ws(int n_tiles, int ks) {
  if (ks <= 1) return 0;
  return ((size_t)n_tiles * 4 + 255) / 256 * 256 + ((size_t)ks * n_tiles * 16 * 4 + 255) / 256 * 256;
}

int plan_ks(int chunks) { return chunks <= 4 * S ? 1 : (chunks + 4 * S - 1) / (4 * S); }

}  // namespace

extern "C" size_t mi_gemv_chain_workspace_bytes(const mi_gemv_desc* phases, int32_t n_phases) {
  if (!phases || n_phases < 1 || n_phases > MAX_PHASES) return 0;
  size_t b = kCtlBytes;
  for (int i = 0; i < n_phases; ++i) {
    if (phases[i].format != MI_FMT_NVFP4 || phases[i].k <= 0 || phases[i].k % 128) return 0;
    const int chunks = phases[i].k / 128;
    b += phase_ws((phases[i].n + 15) / 16, plan_ks(chunks));
  }
  return b;
}

extern "C" int mi_gemv_chain(const mi_gemv_desc* phases, int32_t n_phases, void* workspace, size_t workspace_bytes,
                             void* stream) {
  MI_REQUIRE(phases && n_phases >= 1 && n_phases <= MAX_PHASES, "mi_gemv_chain: 1..%d phases", MAX_PHASES);
  ChainArgs a{};
  a.n_phases = n_phases;
  int max_items = 0;
  for (int i = 0; i < n_phases; ++i) {
    const mi_gemv_desc& d = phases[i];
    MI_REQUIRE(d.format == MI_FMT_NVFP4, "mi_gemv_chain: phase %d: NVFP4 weights only", i);
    MI_REQUIRE(d.m == 1 && !d.groups && !d.out_f32, "mi_gemv_chain: phase %d: one token, dense, BF16 output", i);
    MI_REQUIRE(d.n > 0 && d.k > 0 && d.k % 128 == 0, "mi_gemv_chain: phase %d: k=%d must be a multiple of 128", i, d.k);
    MI_REQUIRE(d.w && d.x && d.y, "mi_gemv_chain: phase %d: null pointer", i);
    MI_REQUIRE(d.epilogue >= MI_EPI_NONE && d.epilogue <= MI_EPI_SILU_MUL_ROUNDED, "mi_gemv_chain: bad epilogue");
    MI_REQUIRE(d.epilogue != MI_EPI_RESIDUAL || d.residual, "mi_gemv_chain: phase %d: residual missing", i);
    MI_REQUIRE(d.epilogue < MI_EPI_SILU_MUL || d.n % 16 == 0, "mi_gemv_chain: phase %d: silu·mul needs n % 16 == 0", i);
    MI_REQUIRE(!(d.norm_w && d.gnorm_w), "mi_gemv_chain: phase %d: one fused norm at most", i);
    MI_REQUIRE(!d.gnorm_w || (d.gnorm_z && d.k % 128 == 0), "mi_gemv_chain: phase %d: gated norm needs z", i);
    MI_REQUIRE((reinterpret_cast<uintptr_t>(d.x) & 15) == 0 && (!d.gnorm_z || (reinterpret_cast<uintptr_t>(d.gnorm_z) & 15) == 0),
               "mi_gemv_chain: phase %d: x and z must be 16-byte aligned", i);
    const int chunks = d.k / 128;
    const int ks = plan_ks(chunks);
    MI_REQUIRE(ks == 1 || !(d.norm_w || d.gnorm_w), "mi_gemv_chain: phase %d: a fused norm needs K <= %d", i, 4 * S * 128);
    MI_REQUIRE(ks <= MAX_KS, "mi_gemv_chain: phase %d: K = %d exceeds %d", i, d.k, MAX_KS * 4 * S * 128);
    Phase& P = a.ph[i];
    P.w = static_cast<const uint8_t*>(d.w);
    P.row_scale = d.row_scale;
    P.x = d.x;
    P.y = d.y;
    P.res = d.residual;
    P.norm_w = d.norm_w;
    P.gnorm_w = d.gnorm_w;
    P.gnorm_z = d.gnorm_z;
    P.ld_gnorm_z = d.ld_gnorm_z;
    P.eps = d.eps;
    P.gnorm_eps = d.gnorm_eps;
    P.n = d.n;
    P.k = d.k;
    P.chunks = chunks;
    P.n_tiles = (d.n + 15) / 16;
    P.ks = ks;
    int kc = (chunks + ks - 1) / ks;
    if (ks > 1) kc = (kc + 7) / 8 * 8;                 // splits on scale-group boundaries
    P.kc = kc;
    P.epilogue = d.epilogue;
    P.items = P.n_tiles * ks;
    P.tile_stride = nv_tile_bytes(chunks);
    max_items = std::max(max_items, P.items);
    // an input or residual written by an earlier phase of this launch is read at the coherence point
    for (int j = 0; j < i; ++j) {
      const mi_gemv_desc& e = phases[j];
      const size_t ybytes = (size_t)((e.epilogue >= MI_EPI_SILU_MUL) ? e.n / 2 : e.n) * 2;
      if (overlaps(d.x, (size_t)d.k * 2, e.y, ybytes)) P.x_chain = 1;
      if (d.residual && overlaps(d.residual, (size_t)d.n * 2, e.y, ybytes)) P.res_chain = 1;
      MI_REQUIRE(!d.gnorm_z || !overlaps(d.gnorm_z, (size_t)d.k * 2, e.y, ybytes),
                 "mi_gemv_chain: phase %d: z must not come from an earlier phase", i);
    }
  }
  const size_t need = mi_gemv_chain_workspace_bytes(phases, n_phases);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = workspace;
  if (ws) {
    MI_REQUIRE(workspace_bytes >= need, "mi_gemv_chain: workspace %zu B < %zu B", workspace_bytes, need);
  } else if (int rc = mi_library_scratch(MI_SCRATCH_CHAIN, need, s, &ws)) {
    return rc;
  }
  char* wb = static_cast<char*>(ws);
  a.ctl = reinterpret_cast<uint32_t*>(wb);
  size_t off = kCtlBytes;
  for (int i = 0; i < n_phases; ++i) {
    Phase& P = a.ph[i];
    if (P.ks > 1) {
      P.fold_cnt = reinterpret_cast<uint32_t*>(wb + off);
      P.part = reinterpret_cast<float*>(wb + off + ((size_t)P.n_tiles * 4 + 255) / 256 * 256);
      off += phase_ws(P.n_tiles, P.ks);
    }
  }
  const int grid = std::max(1, std::min(max_items, cu_count_now() * blocks_per_cu()));
  hipLaunchKernelGGL(gemv_chain, dim3(grid), dim3(64 * S), 0, s, a);
  MI_TRY_HIP(hipGetLastError(), "gemv_chain launch");
  return MI_OK;
}

// the control block's error flag (a wait ran past its bound: the grid could not become resident together)
extern "C" int mi_gemv_chain_error(const void* workspace, void* stream, uint32_t* out) {
  MI_REQUIRE(out, "mi_gemv_chain_error: null output");
  void* ws = const_cast<void*>(workspace);
  if (!ws && mi_library_scratch(MI_SCRATCH_CHAIN, kCtlBytes, static_cast<hipStream_t>(stream), &ws)) return MI_E_HIP;
  MI_TRY_HIP(hipMemcpyAsync(out, static_cast<char*>(ws) + 4 * (MAX_PHASES + 1), 4, hipMemcpyDeviceToHost,
                            static_cast<hipStream_t>(stream)), "hipMemcpyAsync(chain error)");
  // reading the flag clears it (the launches re-arm only their phase counters), so a later read reports later
  // launches only; this call synchronizes its stream, so it is never part of a captured graph
  MI_TRY_HIP(hipMemsetAsync(static_cast<char*>(ws) + 4 * (MAX_PHASES + 1), 0, 4, static_cast<hipStream_t>(stream)),
             "hipMemsetAsync(chain error)");
  MI_TRY_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
  return MI_OK;
}
