/* lithos_mi355.h — the C ABI of the gfx950 (MI355X) decode-layer backend.
 *
 * Everything here is plain C: opaque handles are void*, device memory is void*, sizes are int32/size_t. No torch
 * types cross this boundary. Every function returns 0 (MI_OK) or an MI_E* code; mi_last_error() returns the message
 * of the calling thread's last failure. Work is enqueued asynchronously on the given HIP stream (NULL = the null
 * stream); nothing blocks unless its name says so (…_synchronize, mi_memcpy_d2h on the null stream).
 *
 * Each entry point replaces a piece of the reference's native layer or one of its kernels; the citation names the
 * reference interface (paths relative to lithos-ai/lithos-metal).
 */
#ifndef LITHOS_MI355_H
#define LITHOS_MI355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_OK 0
#define MI_E_INVALID 1     /* bad argument, shape or format: nothing was enqueued */
#define MI_E_HIP 2         /* a HIP runtime call failed */
#define MI_E_UNSUPPORTED 3 /* not built for this device (needs gfx950) */

/* weight storage formats (reference plugin names in monolith/formats/registry.py) */
#define MI_FMT_NVFP4 1       /* "nvfp4": E2M1 codes, E4M3 scale per 16, FP32 tensor scale (formats/nvfp4.py) */
#define MI_FMT_INT4_AFFINE 2 /* "int4_affine": u4 codes, BF16 (scale, bias) per 64 (formats/int4_affine.py) */
#define MI_FMT_BF16 3        /* "bf16": plain BF16 rows (formats/bf16.py) — the router / gate projections */
#define MI_FMT_FP8_E4M3 4    /* "fp8_e4m3": E4M3 codes, FP32 tensor scale (formats/fp8_e4m3.py) — M <= 2, or NVFP4-like
                                dense plans above (no grouped / gated-norm launches) */

/* GEMV epilogues (ops/gemv.py:1-12, nn/linear.py:114-135) */
#define MI_EPI_NONE 0
#define MI_EPI_RESIDUAL 1         /* y = bf16(acc + residual) */
#define MI_EPI_SILU_MUL 2         /* rows are gate|up interleaved by 8: y = bf16(silu(gate)·up), N/2 columns */
#define MI_EPI_SILU_MUL_ROUNDED 3 /* as above with gate and up rounded to BF16 first (nn/moe.py:333-336) */

/* ---- errors / device (runtime/src/metal_core.h:20-35 Device/DeviceInfo; native.mm:13-20) ---------------------- */
const char* mi_version(void);
int mi_last_error(char* buf, size_t n);
typedef struct mi_device_info {
  char name[64];
  char arch[64];         /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t clock_khz;
  int64_t hbm_bytes;
  int32_t lds_bytes_per_block;
  int32_t warp_size;
} mi_device_info;
int mi_device_count(int32_t* count);
int mi_device_info_get(int32_t device, mi_device_info* out);
int mi_set_device(int32_t device);

/* ---- buffers (metal_core.h:37-48 Buffer: alloc / init-from-bytes / read / write / fill) ------------------------- */
int mi_malloc(void** ptr, size_t bytes);
int mi_free(void* ptr);
int mi_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int mi_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int mi_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int mi_memset(void* dst, int32_t byte, size_t bytes, void* stream);

/* ---- streams, timing, graphs (metal_core.mm:128-210 Queue.run/profile; metal_core.h:106-116 Icb) ---------------- */
int mi_stream_create(void** stream);
int mi_stream_destroy(void* stream);
int mi_stream_synchronize(void* stream);
int mi_event_create(void** event);
int mi_event_destroy(void* event);
int mi_event_record(void* event, void* stream);
int mi_event_synchronize(void* event);
int mi_event_elapsed_ms(void* start, void* end, float* ms);
int mi_graph_begin(void* stream);                        /* start capturing the stream's launches (Icb encode) */
int mi_graph_end(void* stream, void** graph_exec);       /* finish capture, instantiate */
int mi_graph_launch(void* graph_exec, void* stream);     /* replay (Icb executeCommandsInBuffer) */
int mi_graph_destroy(void* graph_exec);

/* ---- run-time kernels (metal_core.h:50-66 Library(source, macros) / Pipeline(function); native.mm:42-58
 *      Dispatch; metal_core.mm:95-127). Source compiles with hiprtc for gfx950 into a code object (no GPU needed);
 *      macros are n (name, value) pairs → -Dname=value (an empty value → -Dname). A compile error returns
 *      MI_E_INVALID with the compiler log's tail in mi_last_error. Library and kernel handles are opaque; a kernel
 *      lives as long as its library. mi_launch passes the kernel's parameters as one packed block laid out as the
 *      kernel's parameter list (the HIP kernarg segment), at most 4096 bytes. ------------------------------------ */
typedef struct mi_kernel_attrs {
  int32_t max_threads_per_block, static_lds_bytes, registers, scratch_bytes, wave_size;
} mi_kernel_attrs;
int mi_library_compile(const char* source, const char* const* macros, int32_t n_macros, int32_t fast_math,
                       void** code, size_t* code_bytes);   /* code: malloc'd, release with mi_code_free */
int mi_code_free(void* code);
int mi_library_load(const void* code, size_t code_bytes, void** library);    /* on the current device */
int mi_library_release(void* library);
int mi_kernel_get(void* library, const char* name, void** kernel);          /* "no kernel named …" if absent */
int mi_kernel_info(void* kernel, mi_kernel_attrs* out);
int mi_launch(void* kernel, const void* args, size_t args_bytes, const uint32_t grid[3], const uint32_t block[3],
              uint32_t lds_bytes, void* stream);                            /* grid in workgroups */

/* ---- a file window in device memory (metal_core.mm:70-90 Buffer(path, offset, nbytes): page-aligned offset and
 *      length, as there). Read through a 64 MiB pinned staging buffer; release with mi_free. */
int mi_buf_from_file(const char* path, uint64_t offset, size_t bytes, void** ptr);

/* ---- weight packs ----------------------------------------------------------------------------------------------
 * The T16 pack: 16-row tiles × 128-column chunks (32 for BF16), one 1152-byte unit per (tile, chunk) holding the
 * 64 lanes' 16-byte code words followed by the tile's block scales — the gfx950 counterpart of the reference's
 * block-lane-major pack (formats/blm.py:56-266, PackLayout formats/base.py:10-34). Host code writes it
 * (monolith_mi355/formats/pack.py); mi_pack_bytes gives its size. */
size_t mi_pack_bytes(int32_t format, int32_t n, int32_t k);

/* ---- GEMV / skinny GEMM (ops/gemv.py `gemv`; kernels/common/gemv_T.metal:232-587; kernels.py:222-226 GemvParams;
 *      the M>=2 matrix path kernels/common/gemm_tile.metal:259) and its MoE pairs mode (ops/moe.py `moe_gemv`,
 *      gemv_T.metal:331-358 PAIRS, moe_group.metal + moe_gemm.metal) ------------------------------------------- */
typedef struct mi_gemv_desc {
  int32_t format;            /* MI_FMT_* */
  int32_t n, k;              /* rows and columns of one matrix (one expert in grouped mode) */
  int32_t m;                 /* tokens (dense mode, 1..16); in grouped mode the token count of the step */
  const void* w;             /* T16 pack; grouped mode: n_experts packs back to back */
  const float* row_scale;    /* NVFP4 / FP8 tensor scale per row [experts·n_pad] (the reference's row-scale table); NULL=1 */
  const uint16_t* x;         /* BF16 activations, row stride ldx */
  int32_t ldx;
  uint16_t* y;               /* BF16 output, row stride ldy */
  int32_t ldy;
  int32_t epilogue;          /* MI_EPI_* */
  const uint16_t* residual;  /* BF16 [m, ldr] for MI_EPI_RESIDUAL */
  int32_t ldr;
  const float* norm_w;       /* fused input RMSNorm: x = bf16(h·rsqrt(mean h²+eps)·norm_w), norm_w = (1+w) [k]; NULL = off */
  float eps;
  const int32_t* groups;     /* grouped (MoE) mode: [max_groups][18] = expert, count, 16 pair ids (mi_moe_route);
                                written instead of read when route_logits is set */
  int32_t max_groups;
  int32_t top_k;             /* pair p = token·top_k + slot */
  int32_t x_per_slot;        /* grouped: x row = p (1) or p / top_k (0); y row = p */
  void* workspace;           /* split-K counters + partials (zero it once; reusable by any later GEMV shape, but
                                calls overlapping in time need distinct workspaces); NULL = the library's own */
  size_t workspace_bytes;
  int32_t out_f32;           /* 1: y is FP32 (the lm_head / kernel-test output, ops/gemv.py:12), unrounded */
  /* gated head RMSNorm applied to x while it is staged — the Gated DeltaNet output norm (ops/gdn.py `gdn_norm`,
   * nn/gdn.py:86-93) fused into the output projection: per 128-column head of each x row,
   * x' = bf16(bf16(bf16(w)·bf16(x·r))·silu(z)), r = rsqrt(mean over the head of x² + eps). NVFP4 / INT4 only;
   * exclusive with norm_w. NULL = off. */
  const float* gnorm_w;      /* [128] BF16-valued weights */
  const uint16_t* gnorm_z;   /* z [m][ld_gnorm_z] BF16, same rows as x */
  int32_t ld_gnorm_z;
  float gnorm_eps;
  /* grouped mode: the MoE shared expert stacked after the routed experts (its index, >= 1; 0 = none) runs in the
   * same launch as a group of its own with its own epilogue — the shared expert's gate|up is one BF16 rounding of
   * silu(gate)·up where the routed experts round gate and up first (nn/moe.py:327-337 against nn/mlp.py:25-26) */
  int32_t shared_expert;
  int32_t shared_epilogue;   /* MI_EPI_* for the shared expert's group */
  /* grouped mode at one token (m = 1): the launch routes for itself — the top-k of route_logits (the token's router
   * row: route_experts BF16 logits, the shared gate's logit at route_gate_col), exactly mi_moe_route's — group g is
   * slot g (the shared expert last, when shared_expert > 0; top_k = max_groups = route_top_k (+1)), and its first
   * workgroup writes the route for the launches after it: route_ids / route_weights [top_k] and the group records
   * in `groups` (record g = slot g). NULL = the groups are read from `groups`. No counterpart in the reference: it
   * removes the route launch between the router and the expert GEMVs. */
  const uint16_t* route_logits;
  int32_t route_experts, route_top_k, route_renorm, route_gate_col;
  int32_t* route_ids;
  float* route_weights;
  /* grouped mode: at most this many pairs per record (mi_moe_route's pairs_per_record); 0 = up to 16 */
  int32_t group_max_pairs;
  /* with route_logits: the logits row's width in elements (route_experts <= route_ld; the shared gate's column
   * route_gate_col < route_ld), so the launch never reads past the row */
  int32_t route_ld;
  /* the Gated DeltaNet short causal conv in the input projection's epilogue (dense, m <= 2; no counterpart in the
   * reference, whose conv runs inside gdn_mixer, gdn_mixer.metal:300-420): output rows conv_row0 ..
   * conv_row0 + conv_channels (whole tiles) are the conv's channels q | k | v. Each is convolved over
   * [its W-1 = 3 state inputs | the m new BF16 outputs] with its 4 BF16 taps conv_w [channels][4], as the oracle
   * does (y = Σ w·x in order, then bf16(silu(bf16(y)))), into conv_out [m][ld_conv] (channel order; the step then
   * reads it through mi_gdn_desc.pre), and the new state (the last 3 inputs) goes to the conv state's output slot.
   * State slots as mi_gdn_desc: with conv_step, conv_in holds [2][channels][3], read at slot step & 1 and written
   * at the other (conv_out_state NULL); without, conv_in / conv_out_state name them. conv_done set: no token — the
   * state is copied unchanged and conv_out is not written. conv_w NULL = off. The projection rows are written as
   * usual. */
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out_state;
  uint16_t* conv_out;
  int32_t conv_row0, conv_channels, ld_conv;
  const uint32_t* conv_step;
  const uint32_t* conv_done;
  /* the next RMSNorm of the output, written with it (dense, BF16 output, epilogue none or residual): next_x =
   * bf16(y·rsqrt(mean y² + next_eps)·next_norm_w), next_norm_w = (1+w) [n] — what mi_norm_apply over y gives, bit
   * for bit, and what the next GEMV's M >= 3 input norm computes. Where the plan ends in a split-K reduction launch
   * (M >= 3) that launch computes it, so the next layer's input norm takes no launch of its own; otherwise a norm
   * launch follows the GEMV. No counterpart in the reference (its norms run where they are consumed). NULL = off. */
  const float* next_norm_w;
  uint16_t* next_x;
  int32_t ld_next_x;
  float next_eps;
} mi_gemv_desc;
size_t mi_gemv_workspace_bytes(const mi_gemv_desc* d);   /* 0 when the plan needs none */
int mi_gemv(const mi_gemv_desc* d, void* stream);
/* mi_gemv that allocates nothing — no counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same descriptor, plans and
 * kernels as mi_gemv, with workspace = NULL: split-K plans use one fixed device-resident array per GPU
 * (mi_gemv_noalloc_scratch_bytes(), 8 MiB), and a shape needing more returns MI_E_INVALID. Every call on a GPU shares
 * that GPU's array: calls that overlap in time on one GPU (several streams, or host threads) race. */
int mi_gemv_noalloc(const mi_gemv_desc* d, void* stream);
size_t mi_gemv_noalloc_scratch_bytes(void);
/* the launch plan mi_gemv would use (host only; the tiles per workgroup of a fused-norm M = 1 plan follow the
 * current device's occupancy): out = [kernel (1: gemv_row, the M <= 2 kernel whose waves split a tile's K; 2:
 * gemv_tk, the tile-streaming kernel), waves per workgroup, chunks per wave (row) or chunks per K split (tk),
 * tiles per workgroup, K splits, LDS bytes, workgroups] */
int mi_gemv_plan(const mi_gemv_desc* d, int32_t out[7]);

/* A chain of dependent one-token NVFP4 GEMVs in ONE persistent launch — a decode layer's projection tail
 * (out_proj → gate|up → down, or the MLP's gate|up → down): the counterpart of the reference's region / MLP fusion
 * into a megakernel with bounded worker synchronization (compiler/region_fusion.py:25-58, compiler/mlp_fusion.py:103-130,
 * runtime/engine.py:100-105). Phase i is phases[i] with mi_gemv's semantics (m = 1, dense, BF16 output, fused input
 * RMSNorm or gated head norm, residual / silu·mul epilogues; K up to 6144 with a fused norm, longer K split in order)
 * and starts only after phase i-1 has finished, so it may read any earlier phase's output (as x or residual).
 * workspace: mi_gemv_chain_workspace_bytes, zeroed once before its first use (its counters return to zero after every
 * launch); NULL = the library's own. mi_gemv_chain_error reads the control block's error flag (1: a wait ran past its
 * bound because the grid could not run together; the results are then wrong) and clears it, so each read reports the
 * launches since the previous read. */
#define MI_CHAIN_MAX_PHASES 4
size_t mi_gemv_chain_workspace_bytes(const mi_gemv_desc* phases, int32_t n_phases);
int mi_gemv_chain(const mi_gemv_desc* phases, int32_t n_phases, void* workspace, size_t workspace_bytes, void* stream);
int mi_gemv_chain_error(const void* workspace, void* stream, uint32_t* out);

/* exact dequantization of a T16 pack to FP32 [n, k] through the kernels' own decode (the bit-exact check of
 * Format.dequantize, formats/base.py:52-81 / nvfp4.py:139-144 / int4_affine.py:85-91) */
int mi_dequant(int32_t format, const void* w, const float* row_scale, int32_t n, int32_t k, float* out, void* stream);

/* ---- RMSNorm as standalone ops (ops/norm.py:11-12: rmsnorm_stat, norm_apply; kernels/common/rmsnorm_stat.metal:18-40,
 *      norm_apply.metal:24-51) — for a norm that does not feed a GEMV directly (mi_gemv fuses it on load) ----------
 * rmsnorm_stat: stat[i] = Σ_k h[i][k]² (FP32). norm_apply: x[i] = bf16(h[i]·rsqrt(s/k + eps)·w), s = Σ of the
 * stat_parts partial sums stat[i][·], or — with stat = NULL — computed in the same launch; w is the (1 + w) weight.
 * h and x: BF16 rows, 16-byte aligned, strides multiples of 8, k a multiple of 8. */
typedef struct mi_norm_desc {
  int32_t t, k;
  const uint16_t* h;
  int32_t ldh;
  float* stat;               /* rmsnorm_stat: output [t]; norm_apply: input [t][stat_parts] or NULL */
  int32_t stat_parts;
  const float* w;            /* norm_apply: (1 + w) [k] FP32 */
  uint16_t* x;               /* norm_apply: output [t][ldx] */
  int32_t ldx;
  float eps;
} mi_norm_desc;
int mi_rmsnorm_stat(const mi_norm_desc* d, void* stream);
int mi_norm_apply(const mi_norm_desc* d, void* stream);

/* ---- Gated DeltaNet decode step (ops/gdn.py `gdn_mixer` + `gdn_norm`; nn/gdn.py:64-93;
 *      kernels/common/gdn_mixer.metal:272-589; GdnParams kernels.py:686-720) ------------------------------------
 * proj holds the in-projection output of T tokens: z | q | k | v | a | b at the given column offsets (a|b may sit
 * in a second buffer). conv_in/conv_out: the causal-conv state [2·hk·dk + hv·dv][W-1] BF16, channel order q|k|v
 * (distinct buffers: ping-pong them by step parity); rec_in/rec_out: the recurrent state [hv][dk][dv] FP32 (may
 * alias). y [T][hv·dv] BF16 = the gated RMSNorm output. Built for dk = dv = 128, W = 4, T <= 16. */
typedef struct mi_gdn_desc {
  int32_t t, k_heads, v_heads, dk, dv, conv_width;
  const uint16_t* proj;
  int32_t ld_proj, z_off, q_off, k_off, v_off;
  const uint16_t* ab;        /* NULL: a|b are in proj */
  int32_t ld_ab, a_off, b_off;
  const uint16_t* conv_w;    /* [conv_dim][W] BF16 */
  const float* neg_exp_a;    /* [hv] −exp(A_log) (the pack's transform, packs/transforms.py:595-598) */
  const float* dt_bias;      /* [hv] */
  const float* norm_w;       /* [dv] BF16-valued gated-norm weight */
  const uint16_t* conv_in;
  uint16_t* conv_out;
  const float* rec_in;
  float* rec_out;
  uint16_t* y;
  int32_t ld_y;
  float eps;
  int32_t defer_norm;        /* 1: y gets the BF16 read-out o and the gated RMSNorm is left to the consumer (the
                                output projection's mi_gemv, gnorm_* fields); 0: y is the normed, gated output */
  int32_t commit;            /* 1: the speculative commit pass (ops/gdn.py `gdn_commit`, gdn_mixer.metal:331-347):
                                replay the committed tokens from the step's input state rec_in into rec_out (the same
                                slot, in place, or another); no read-out (y may be NULL) */
  const int32_t* t_dev;      /* device-resident token count 0..t (the accept scan's committed count), or NULL = t */
  const uint32_t* done;      /* a step program's mi_step_state.done, or NULL: once it is set the step takes no token —
                                conv_out and rec_out receive conv_in and rec_in unchanged (so a graph's fixed ping-pong
                                stays in phase) and y is not written (gdn_mixer.metal:281,330 return at done) */
  const uint32_t* step;      /* a step program's mi_step_state.step, or NULL. Set: the conv state is two slots
                                [2][conv_dim][W-1] at conv_in (conv_out = NULL), chosen by the step's parity — read
                                slot step & 1, write the other (gdn_mixer.metal:25-37's SLOTS = 2); the commit pass
                                runs after the accept scan advanced step, so it reads slot (step + 1) & 1 */
  /* the conv already done by the input projection (mi_gemv_desc.conv_*): pre [t][ld_pre] holds the convolved,
   * SiLU'd q | k | v channels (BF16, channel order) and the step reads them instead of running the conv; the conv
   * state is then the projection's business (conv_in / conv_out unused, may be NULL). Not with commit. NULL = off */
  const uint16_t* pre;
  int32_t ld_pre;
} mi_gdn_desc;
int mi_gdn_step(const mi_gdn_desc* d, void* stream);

/* ---- GQA decode attention over an int8 or BF16 KV cache (ops/attention.py `gqa_decode` + `gqa_merge`;
 *      nn/attention.py:215-243; kernels/common/gqa_decode.metal:32-302; GqaParams kernels.py:604-611) ----------
 * proj [T][heads·(gate ? 2 : 1)·D + 2·kv·D] BF16 in checkpoint column order (q|gate per head, then k, v). The new
 * tokens are normed (qk_norm), roped (cos/sin [ctx_max][rotary_dim] BF16, cat(freqs, freqs)) and appended at
 * pos..pos+T. Cache (this backend's layout): k_codes [kv][ctx_max][D], v_codes [kv][ctx_max/64][D][64] (transposed
 * inside 64-key blocks), both int8 codes with k_scales / v_scales [kv][ctx_max] f16 bits (scale = f16(absmax/127)
 * per token and KV head) when kv_dtype = MI_KV_INT8, or BF16 values (the reference's cache, nn/attention.py:87-89;
 * the scale pointers unused) when kv_dtype = MI_KV_BF16; ctx_max a multiple of 64.
 * y [T][heads·D] BF16 (× bf16(σ(gate)) when gate). D = 128 or 256, T <= 16, heads/kv·T <= 64 rows per KV head. */
enum { MI_KV_INT8 = 0, MI_KV_BF16 = 1 };
typedef struct mi_gqa_desc {
  int32_t t, heads, kv_heads, head_dim, rotary_dim, pos, ctx_max, gate, qk_norm;
  const uint16_t* proj;
  int32_t ld_proj;
  const uint16_t* rope_cos;
  const uint16_t* rope_sin;
  const float* q_norm;       /* (1 + w) [D], or NULL */
  const float* k_norm;
  float eps, scaling;
  void* k_codes;             /* int8 codes or BF16 values, per kv_dtype */
  uint16_t* k_scales;
  void* v_codes;
  uint16_t* v_scales;
  uint16_t* y;
  int32_t ld_y;
  void* workspace;           /* key-range partials, prepared query rows and the per-KV-head arrival counters of the
                                in-launch merge (mi_gqa_workspace_bytes; zero it once before its first use: the
                                counters return to zero after every call; calls overlapping in time need distinct
                                workspaces); NULL = the library's own */
  size_t workspace_bytes;
  const int32_t* pos_dev;    /* device-resident position (a step program's mi_step_state.position) or NULL = pos;
                                the key ranges are then planned for ctx_max - t and the kernels read the position */
  const uint32_t* done;      /* a step program's mi_step_state.done, or NULL: once it is set nothing is appended to
                                the cache and y is not written (gqa_decode.metal:53,239 return at done) */
  int32_t kv_dtype;          /* MI_KV_INT8 (0) or MI_KV_BF16 (1) */
  /* the reference's packed projection (nn/attention.py:52-64, 133-155): proj holds q | k | v (q heads·D columns)
   * and the gate rows come from their own buffer [T][ld_gate] (the sibling GEMV's output); NULL = the checkpoint
   * order above. The RoPE head-dim permutation of that layout is rotary_dim = head_dim with the permuted tables. */
  const uint16_t* gate_src;
  int32_t ld_gate;
} mi_gqa_desc;
size_t mi_gqa_workspace_bytes(const mi_gqa_desc* d);
int mi_gqa_decode(const mi_gqa_desc* d, void* stream);

/* ---- MoE routing and combine (ops/moe.py `moe_route`, `moe_combine`; nn/moe.py:108-135;
 *      kernels/common/moe_route.metal:20-66, moe_combine.metal:19-49, moe_group.metal:8-47) -----------------------
 * Route: logits [t][ld_logits] BF16 → ids [t][top_k] int32, weights [t][top_k] float (BF16-valued): softmax in FP32,
 * top-k with ties to the lowest expert index, renormalized over the k when renorm. With `groups` non-NULL the same
 * launch writes the expert groups of the grouped GEMV (mi_gemv_desc.groups): max_groups records of 18 int32 —
 * expert, count, then the count pair ids p = t·top_k + slot ascending — one per distinct expert in order of first
 * use, the rest expert = -1, count = 0. t <= 16, n_experts <= 512, top_k <= 16.
 * shared_expert > 0: the shared expert joins every token as slot top_k — id shared_expert, weight
 * bf16(σ(logits[t][shared_gate_col])) (the shared gate's logit, a row of the router GEMV) — so ids / weights are
 * [t][top_k + 1], pairs p = t·(top_k + 1) + slot, and the shared expert is one more group (max_groups one more). */
typedef struct mi_moe_route_desc {
  int32_t t, n_experts, top_k, renorm;
  const uint16_t* logits;
  int32_t ld_logits;
  int32_t* ids;
  float* weights;
  int32_t* groups;
  int32_t max_groups;
  int32_t shared_expert;     /* 0 = none */
  int32_t shared_gate_col;
  /* 1..16: an expert's pairs go into consecutive records of at most this many (max_groups >= t·slots), so a grouped
   * GEMV that takes two pairs per workgroup needs one pass per record; 0 = one record per expert (up to 16 pairs).
   * No counterpart in the reference (its groups are per expert). */
  int32_t pairs_per_record;
} mi_moe_route_desc;
int mi_moe_route(const mi_moe_route_desc* d, void* stream);

/* Combine: out[t] = Σ_j w[t][j]·h[t·top_k + j] (+ bf16(σ(shared_gate[t]))·shared[t]) (+ residual[t]), FP32, one BF16
 * rounding. h [t·top_k][ldh], shared [t][ld_shared], shared_gate [t] at stride ld_gate, residual [t][ldr], out [t][ldo],
 * all BF16; hidden and the row strides multiples of 8, rows 16-byte aligned. shared/shared_gate/residual may be NULL. */
typedef struct mi_moe_combine_desc {
  int32_t t, hidden, top_k;
  const uint16_t* h;
  int32_t ldh;
  const float* weights;
  const uint16_t* shared;
  int32_t ld_shared;
  const uint16_t* shared_gate;
  int32_t ld_gate;
  const uint16_t* residual;
  int32_t ldr;
  uint16_t* out;
  int32_t ldo;
  /* the next RMSNorm of out, written with it: next_x = bf16(out·rsqrt(mean out² + next_eps)·next_norm_w), bit for
   * bit mi_norm_apply over out (hidden <= 8192: one workgroup per token computes both). No counterpart in the
   * reference. NULL = off. */
  const float* next_norm_w;
  uint16_t* next_x;
  int32_t ld_next_x;
  float next_eps;
} mi_moe_combine_desc;
int mi_moe_combine(const mi_moe_combine_desc* d, void* stream);

/* ---- The GPU-resident token loop (runtime/engine.py:47-122, core/step_state.py:28-73, ops/embed.py, ops/sample.py
 *      `argmax`, the advance op of runtime/src/metal_core.mm:256-386) ------------------------------------------------
 * A step program replays one captured step (embed → layers → final norm + lm_head → argmax → advance) as a HIP graph;
 * everything that changes between steps lives in mi_step_state in device memory, written by the serial ops at the
 * end of the step, so the graph never changes. Emitted tokens go to a ring in pinned host memory as
 * (sequence << 32) | token; the host drains it between launches. */
#define MI_STEP_T_MAX 16
#define MI_STEP_GAMMA_MAX 15
/* Field order and meaning are the reference's StepStateLayout (core/step_state.py:38-63) at t_max = 16,
 * gamma_max = 15: every field a 4-byte scalar or an array of them, 272 bytes. */
typedef struct mi_step_state {
  uint32_t step;                               /* steps completed */
  uint32_t position;                           /* position of the first token of this step */
  uint32_t kv_len;                             /* committed context length */
  uint32_t t_this_step;                        /* tokens in this step */
  int32_t pending_tokens[MI_STEP_T_MAX];       /* token ids fed to this step (embed reads them) */
  uint32_t rng_lo, rng_hi;
  int32_t anchor;
  uint32_t gamma;
  int32_t draft_tokens[MI_STEP_GAMMA_MAX];
  float confidence[MI_STEP_GAMMA_MAX];
  uint32_t verify_len, accepted, checkpoint_index, drafter_ctx_len;
  uint32_t done;                               /* stop condition met: later steps' serial ops do nothing */
  uint32_t error;                              /* 1 token ring overflow, 2 context capacity reached */
  uint32_t ring_head;                          /* next ring slot the GPU writes */
  uint32_t ring_tail;                          /* next slot the host reads (host-written) */
  uint32_t prefill_left;                       /* prompt chunks still to feed; the advance emits only at 0 */
  uint32_t n_inject;
  uint32_t stop_at;                            /* host-written: ring head at which done is set (0 = never) */
  uint32_t n_chain;
  uint32_t pad_[2];
} mi_step_state;

/* embed (ops/embed.py:1-7, kernels/common/embed.metal): out[i] = table[tokens[i]] for i < t, BF16 [vocab][hidden]
 * rows; an id outside [0, vocab) reads row 0 */
typedef struct mi_embed_desc {
  int32_t t, vocab, hidden;
  const int32_t* tokens;      /* device: usually mi_step_state.pending_tokens */
  const uint16_t* table;
  uint16_t* out;
  int32_t ldo;
  int32_t t16;                /* 1: table is a BF16 T16 weight slab (the pack's embedding, nn/embedding.py:31-37's
                                 `packed`): a row is gathered from its tile's 32-column chunks; 0: row-major */
} mi_embed_desc;
int mi_embed(const mi_embed_desc* d, void* stream);

/* argmax (ops/sample.py:1-9, kernels/common/argmax.metal): ids[i] = the index of the largest logit of row i; ties →
 * the lowest index; NaN never wins; a row with no number gives -1 */
typedef struct mi_argmax_desc {
  int32_t t, vocab;
  const void* logits;
  int32_t ld, f32;            /* f32: 1 FP32 logits, 0 BF16 */
  int32_t* ids;               /* device [t] */
  void* workspace;            /* optional device buffer of mi_argmax_workspace_bytes, zeroed once before its first use
                                 (its arrival counters return to zero after every call); NULL: the library's own */
  size_t workspace_bytes;
} mi_argmax_desc;
size_t mi_argmax_workspace_bytes(const mi_argmax_desc* d);
int mi_argmax(const mi_argmax_desc* d, void* stream);

/* sample (ops/sample.py:1-10, kernels/common/sample.metal, nn/sampling_ref.py): per row of BF16 logits, the token
 * argmax over the kept logits (v >= tau) of v / temperature − log(−log u), u from a splitmix64 hash of (seed, step,
 * row, index); tau = the most restrictive of top-k (k-th largest, ties kept; top_k > 0), top-p (0 < top_p < 1: the
 * value where the descending cumulative softmax mass first reaches top_p — of the top-k set with topp_in_topk) and
 * min-p (min_p > 0: max + temperature · log(min_p)). temperature > 0 (greedy is mi_argmax). With state set, the seed
 * is (rng_hi << 32 | rng_lo) and the step is state->step, read on the device. */
typedef struct mi_sample_desc {
  int32_t t, vocab;
  const uint16_t* logits;     /* device BF16 [t][ld] */
  int32_t ld;
  int32_t* ids;               /* device [t] */
  float temperature, top_p, min_p;
  int32_t top_k, topp_in_topk;
  uint64_t seed;
  uint32_t step;
  const mi_step_state* state; /* optional: seed and step from the step state */
  void* workspace;            /* optional, mi_sample_workspace_bytes, zeroed once before its first use (the
                                 histograms and counters are left at zero by every call); NULL: the library's own */
  size_t workspace_bytes;
} mi_sample_desc;
size_t mi_sample_workspace_bytes(const mi_sample_desc* d);
int mi_sample(const mi_sample_desc* d, void* stream);

/* advance (kernels/common/advance.metal:15-37): the serial op that closes a step. Unless done: while prefill_left > 0
 * only position += t_this_step and step += 1; otherwise the last row's token (tokens[t_this_step - 1]) goes to ring
 * slot head % ring_cap as ((head + 1) << 32) | token (ring full: error 1 + done, nothing else changes), becomes
 * pending_tokens[0], position += t_this_step, step += 1, t_this_step = 1; done at the ring head stop_at, at an EOS
 * token, and (error 2) when ctx_cap > 0 and the new position reaches it. */
typedef struct mi_advance_desc {
  mi_step_state* state;       /* device */
  const int32_t* tokens;      /* device: the argmax ids of this step */
  uint64_t* ring;             /* pinned host memory (mi_host_alloc), ring_cap slots */
  uint32_t ring_cap, ctx_cap;
  int32_t n_eos, eos[8];      /* the EOS token ids (n_eos = 0: none) */
  uint32_t* host_ctl;         /* optional pinned host words: [0] the host's ring tail (host-written), [1] done and
                                 [2] error (written by every advance so the host polls them without a copy) */
} mi_advance_desc;
int mi_advance(const mi_advance_desc* d, void* stream);

/* verify_select (kernels/common/spec_ops.metal:108-146): one thread. Unless done: the drafter's context grows by the
 * injected rows (lm: becomes position + gamma, or position in a prefill chunk), n_inject = 0; outside a prefill chunk
 * the block's drafts and confidences go into the state (and conf_log[(step % log_cap) * 16 + k] when log_cap > 0),
 * and the verify length L ≤ min(gamma, t_max − 1) (and ≤ ctx_cap − position − 1; position ≥ ctx_cap: error 2 + done)
 * is chosen — mode 0: the leading drafts with confidence ≥ threshold (threshold ≤ 0: all), mode 1: argmax over l of
 * (1 + Σ_{i≤l} Π_{j≤i} c_j) / cost[l], mode 2: L = threshold — then pending_tokens = [anchor, d_0 … d_{L−1}],
 * t_this_step = 1 + L, gamma and verify_len recorded. */
typedef struct mi_verify_select_desc {
  mi_step_state* state;       /* device */
  const int32_t* drafts;      /* device [gamma] */
  const float* conf;          /* device [gamma] */
  uint32_t gamma, t_max, mode;
  float threshold;
  float cost[16];
  float* conf_log;            /* device [log_cap][16], optional */
  uint32_t log_cap, ctx_cap, lm;
} mi_verify_select_desc;
int mi_verify_select(const mi_verify_select_desc* d, void* stream);

/* accept_scan (kernels/common/spec_ops.metal:148-195): one thread, the closing serial op of a speculative step (in
 * place of the advance). Unless done: a prefill chunk advances the position by t_this_step and marks its rows for
 * injection; otherwise the target's tokens are compared with the drafts the step fed (pending_tokens =
 * [prompt tail …, anchor, d_0 … d_{L−1}], base = t − 1 − L): the matching prefix and the bonus token after it go to
 * the ring (stopping after the first EOS; not enough ring room: error 1 + done, nothing written), position advances
 * by base + committed, anchor = the last committed token, n_inject = checkpoint_index = base + committed (lm: the
 * committed rows the drafter has not seen), verify_len = 0, t_this_step = 1; log[step % log_cap] = (committed << 16)
 * | (L << 8) | accepted ((t << 16) | 0xFFFF for a prefill chunk); done at EOS / stop_at, error 2 at ctx_cap. */
typedef struct mi_accept_scan_desc {
  mi_step_state* state;       /* device */
  const int32_t* tokens;      /* device: the target's argmax per row */
  uint64_t* ring;             /* pinned host, ring_cap slots */
  uint32_t ring_cap, ctx_cap, lm;
  int32_t n_eos, eos[8];
  uint32_t* log;              /* device [log_cap], optional */
  uint32_t log_cap;
  uint32_t* host_ctl;         /* optional pinned host words, as for mi_advance */
} mi_accept_scan_desc;
int mi_accept_scan(const mi_accept_scan_desc* d, void* stream);

/* The host pump (runtime/src/metal_core.mm:256-386 `Runner::run` / `drain`): replay a captured step graph up to
 * max_launches times, launches_per_batch per batch with at most in_flight batches queued; after each completed batch
 * drain the ring by sequence tag into tokens[] and publish the tail (host_ctl[0], copied into state->ring_tail ahead
 * of every batch); stop submitting once host_ctl[1] (done) is set, max_tokens tokens arrived (0 = no limit) or the
 * token buffer is full. n_tokens counts what tokens[] holds (in: already there; out: after the run). */
typedef struct mi_runner_desc {
  void* graph_exec;           /* from mi_graph_end */
  void* stream;
  mi_step_state* state;       /* device */
  const uint64_t* ring;       /* pinned host (mi_host_alloc) */
  uint32_t ring_capacity;
  uint32_t* host_ctl;         /* pinned host, the words the advance writes */
  uint32_t max_launches, launches_per_batch, in_flight;
  uint64_t max_tokens;
  int32_t* tokens;            /* host */
  uint64_t tokens_capacity, n_tokens;
  /* optional, for a step state held in pinned host memory in a program's own layout (Engine programs): the runner
   * stores the tail into state_ring_tail (instead of copying it into state->ring_tail) and reads done / error from
   * state_done / state_error (instead of host_ctl[1] / [2]); state may then be NULL. host_ctl[0] keeps the tail. */
  uint32_t* state_ring_tail;
  const uint32_t* state_done;
  const uint32_t* state_error;
} mi_runner_desc;
typedef struct mi_runner_stats {
  uint64_t launches, batches, tokens;
  double wall_ms, gpu_ms, launch_ms, wait_ms, host_busy_ms;
  uint32_t done, error;
} mi_runner_stats;
int mi_runner_run(mi_runner_desc* d, mi_runner_stats* stats);

/* pinned, device-accessible host memory for the token ring (hipHostMalloc); freed with mi_host_free */
void* mi_host_alloc(size_t bytes);
int mi_host_free(void* p);

#ifdef __cplusplus
}
#endif
#endif /* LITHOS_MI355_H */
