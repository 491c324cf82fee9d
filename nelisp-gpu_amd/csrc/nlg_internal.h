// nlg_internal.h -- shared declarations of libnlgpu's HIP translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nlgpu.h"

// ---------------------------------------------------------------- host side

// Record a failure message for nlg_last_error(); always returns NLG_ERR.
int nlg_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
// NULL -> the library stream.  Requires nlg_init() (done lazily).
hipStream_t nlg_stream(void *s);
// Ensure the device is initialised (nlg_init(-1) on first use).
int nlg_ensure_init(void);
int nlg_num_cu(void);

#define NLG_HIP(call)                                                              \
  do {                                                                             \
    hipError_t _e = (call);                                                        \
    if (_e != hipSuccess)                                                          \
      return nlg_fail("%s failed: %s (%s:%d)", #call, hipGetErrorString(_e),     \
                      __FILE__, __LINE__);                                         \
  } while (0)

// Check a launch that just happened.
#define NLG_LAUNCHED(what)                                                         \
  do {                                                                             \
    hipError_t _e = hipGetLastError();                                             \
    if (_e != hipSuccess)                                                          \
      return nlg_fail("launch of %s failed: %s", (what), hipGetErrorString(_e));   \
  } while (0)

// A kernel reachable by name: validates buffers against the extents its
// push constants imply, then launches on `st`.
typedef int (*nlg_launcher)(const nlg_buffer *b, const uint32_t *p, uint32_t groups,
                            hipStream_t st);

// Buffer i must hold at least `need` elements (need computed in 64 bits).
int nlg_need(const nlg_buffer *b, int i, uint64_t need, const char *kname);

// min(domain, 64*groups): how many invocations of a local-64 kernel do work.
static inline uint64_t nlg_domain(uint64_t domain, uint32_t groups, uint32_t local = 64) {
  uint64_t lim = (uint64_t)groups * local;
  return domain < lim ? domain : lim;
}

// grid size for n items with `per` items per block, at least 1.
static inline uint32_t nlg_blocks(uint64_t n, uint64_t per) {
  uint64_t b = (n + per - 1) / per;
  if (b == 0) b = 1;
  if (b > 0x7fffffffull) b = 0x7fffffffull;
  return (uint32_t)b;
}

// ---------------------------------------------------------------- device side

// (uint f) of the DSL: OpConvertFToS into a uint (lisp/nelisp-gpu-compile.el:327).
// Truncation toward zero; NaN -> 0 and out-of-range saturates (undefined in
// SPIR-V; the CPU restatement uses the same convention).
__device__ __forceinline__ uint32_t nlg_f2u(float f) {
  if (!(f == f)) return 0u;
  if (f >= 2147483648.0f) return 0x7fffffffu;
  if (f <= -2147483648.0f) return 0x80000000u;
  return (uint32_t)(int32_t)f;
}

// Wave64 reductions on DPP.  Lanes 0..63 must all be active.  Each returns
// the full-wave result in every lane (read back from lane 63).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int nlg_dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}

// A quad permutation (every source lane exists, so no fill value is needed:
// no zeroing move ahead of the DPP move).
template <int CTRL>
__device__ __forceinline__ uint32_t nlg_qperm(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}

__device__ __forceinline__ int nlg_wave_sum_i32(int v) {
  v += nlg_dpp<0xB1>(v);        // quad_perm [1,0,3,2]
  v += nlg_dpp<0x4E>(v);        // quad_perm [2,3,0,1]
  v += nlg_dpp<0x124>(v);       // row_ror:4
  v += nlg_dpp<0x128>(v);       // row_ror:8   -> every lane holds its row's sum
  v += nlg_dpp<0x142, 0xa>(v);  // row_bcast:15 into rows 1,3
  v += nlg_dpp<0x143, 0xc>(v);  // row_bcast:31 into rows 2,3
  return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ float nlg_fdpp_add(float v, int x) { return v + __int_as_float(x); }

__device__ __forceinline__ float nlg_wave_sum_f32(float v) {
  v = v + __int_as_float(nlg_dpp<0xB1>(__float_as_int(v)));
  v = v + __int_as_float(nlg_dpp<0x4E>(__float_as_int(v)));
  v = v + __int_as_float(nlg_dpp<0x124>(__float_as_int(v)));
  v = v + __int_as_float(nlg_dpp<0x128>(__float_as_int(v)));
  v = v + __int_as_float(nlg_dpp<0x142, 0xa>(__float_as_int(v)));
  v = v + __int_as_float(nlg_dpp<0x143, 0xc>(__float_as_int(v)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over the wave of values that are never NaN; lanes in rows masked off by
// the broadcast steps receive 0 from the DPP move, so the identity used for
// those steps must be handled: callers pass values >= `floor` and floor is
// what masked lanes compare against.
__device__ __forceinline__ float nlg_fmax_nn(float a, float b) { return b > a ? b : a; }

// The split decode attention keeps its scores in base 2: s * log2(e), so
// that every exponential is one v_exp_f32 (exp(s - m) = 2^(s2 - m2)); the
// chunk maxima it leaves for the merges are in the same units.
#define NLG_LOG2E 1.4426950408889634f
__device__ __forceinline__ float nlg_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// silu-mul's gate sg = 1/(1 + exp(0 - g)) (kernels.el:186-193) in the fused
// epilogues: one v_exp_f32 and one v_rcp_f32 (relative error ~1e-6 at
// |g| = 20, well inside the 1e-4 SwiGLU tolerance) in place of a correctly
// rounded expf and division (~25 instructions, most of the prefill GEMM's
// SwiGLU epilogue).
__device__ __forceinline__ float nlg_silu_gate(float g) {
  return __builtin_amdgcn_rcpf(1.0f + nlg_exp2((0.0f - g) * NLG_LOG2E));
}

// A 16-byte load of data streamed once per launch (2-bit weights): marked
// non-temporal (glc slc), so it neither allocates in the caches nor evicts
// the activations and KV rows later kernels re-read.  Measured: the 4096^2
// GEMV 3.24 -> 2.94 us, a B=1 decode step 1.007 -> 0.955 ms.
__device__ __forceinline__ uint4 nlg_ld_stream(const uint4 *p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u t = __builtin_nontemporal_load((const v4u *)p);
  return make_uint4(t.x, t.y, t.z, t.w);
}

// A buffer resource over `bytes` bytes at p (raw, unswizzled; the gfx9
// descriptor word 3): loads through it at offsets past the end read 0
// instead of faulting, so edge lanes need no clamped address.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t nlg_buffer_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// A device-resident int32 that the kernel does not write (the decode
// position), read with a scalar load from the constant address space.  Its
// wait counts scalar loads only, so code that needs it early (RoPE table
// addresses) no longer waits for every vector load issued before it -- the
// weights' whole HBM fetch.  The scalar cache is invalidated at every
// dispatch, so a value written by an earlier kernel is seen.
__device__ __forceinline__ int32_t nlg_ld_uniform_i32(const int32_t *p) {
  return *(const __attribute__((address_space(4))) int32_t *)p;
}

// The same for rows read and written once (softmax in place: 5.49 -> 6.03 TB/s).
__device__ __forceinline__ float4 nlg_ld_stream_f4(const float4 *p) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  const v4f t = __builtin_nontemporal_load((const v4f *)p);
  return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void nlg_st_stream_f4(float4 *p, float4 v) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  const v4f t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, (v4f *)p);
}

__device__ __forceinline__ float nlg_wave_max_f32(float v) {
  // rotations keep every lane valid, so no identity is needed for them
  v = nlg_fmax_nn(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xf, 0xf, false)));
  v = nlg_fmax_nn(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xf, 0xf, false)));
  v = nlg_fmax_nn(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x124, 0xf, 0xf, false)));
  v = nlg_fmax_nn(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x128, 0xf, 0xf, false)));
  // masked rows keep `old` = their own value, so max(v, v) = v there
  v = nlg_fmax_nn(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = nlg_fmax_nn(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Block-wide (blockDim.x multiple of 64, <= 1024) sum / max through LDS.
// `scratch` needs blockDim.x/64 floats.  Every thread gets the result.
// NW > 0 states the block's wave count at compile time (no read of the
// launch's block size).
// FRESH: `scratch` has not been used before in this kernel, so the barrier
// that guards its reuse is left out.
template <int NW = 0, bool FRESH = false>
__device__ __forceinline__ float nlg_block_sum_f32(float v, float *scratch) {
  v = nlg_wave_sum_f32(v);
  const int nw = NW > 0 ? NW : (int)(blockDim.x >> 6), w = threadIdx.x >> 6;
  if (!FRESH) __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < nw; i++) t = t + scratch[i];
  return t;
}
template <int NW = 0, bool FRESH = false>
__device__ __forceinline__ float nlg_block_max_f32(float v, float *scratch) {
  v = nlg_wave_max_f32(v);
  const int nw = NW > 0 ? NW : (int)(blockDim.x >> 6), w = threadIdx.x >> 6;
  if (!FRESH) __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  float t = scratch[0];
  for (int i = 1; i < nw; i++) t = nlg_fmax_nn(t, scratch[i]);
  return t;
}

// ------------------------------------------------- fused quantise + GEMV
// One launch: optional RMSNorm of the activation row, pack-act-rows'
// quantisation into LDS, the 2-bit x int8 GEMV, and an epilogue.
enum {
  NLG_PRO_NONE = 0,  // x as given
  NLG_PRO_RMS = 1,   // x = rmsnorm(x) * gain
  NLG_PRO_ATTN = 2,  // x = decode attention merged from its chunk partials
  // kernel-internal: NLG_PRO_ATTN over exactly 3 chunks (decode at 512 < max_seq <= 768)
  NLG_PRO_ATTN3 = 3,
};
// Most attention chunks the PRO_ATTN prologue merges, and how many chunks
// the decode attention splits max_seq positions into.
#define NLG_ATTN_MAX_CHUNKS 4
uint32_t nlg_attn_chunk_count(uint32_t head_dim, uint32_t max_seq);
// The chunk pass over `rows` query rows: decode (qper 0: row = sequence, all
// at position pos[0]) or prefill (row r = sequence r / qper at position
// pos[0] + r % qper, causal over the cache).  Workspace sized for `rows`.
int nlg_attn_chunks(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos, uint32_t rows,
                    uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                    void *workspace, size_t workspace_bytes, hipStream_t st);
// Causal attention of `rows` prompt rows (row r = sequence r / qper at
// position pos[0] + r % qper) over the fp16 caches on the matrix cores;
// ctx [rows][heads * head_dim] f32, normalised.
// With xq, gamma and quantized given, a launch that splits the keys leaves
// the merged context quantised for the output projection in xq ([rows x
// heads*head_dim] int8 in matrix-core order) and gamma ([rows]) instead of
// ctx, and sets *quantized; otherwise ctx is written as without them.
// pos_bound (0: none) bounds the positions any row attends (pos[0] + qper
// when the caller knows pos[0]), which sizes the split form's workspace.
int nlg_prefill_attn(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos, uint32_t rows,
                     uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                     float *ctx, hipStream_t st, uint8_t *xq = nullptr, float *gamma = nullptr,
                     bool *quantized = nullptr, uint32_t pos_bound = 0);
// Prompt attention + output projection + residual (the stack's prefill
// form; nlg_prefill_attn_ternary_linear_residual in the C ABI).
int nlg_prefill_attn_o_resid(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos,
                             uint32_t rows, uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                             uint32_t max_seq, uint32_t pos_bound, float *ctx_ws, const uint32_t *w2,
                             const float *bias, const float *beta, int beta_per_row, const float *res, float *y,
                             uint32_t out, hipStream_t st);
enum {
  NLG_EPI_STORE = 0,   // y = bias + (beta*gamma)*acc
  NLG_EPI_RESID = 1,   // y = res + that
  NLG_EPI_SWIGLU = 2,  // rows 2j, 2j+1 = gate j, up j; y[j] = silu(gate)*up
  NLG_EPI_QKV = 3,     // rows = q | k | v; RoPE on q, k; k, v appended to fp16 caches
  NLG_EPI_ARGMAX = 4,  // y = logits, plus one (max, index) per wave
  // kernel-internal: NLG_EPI_STORE with no bias, a per-tensor beta and no
  // gamma output (the bare linear: no per-row operand loads)
  NLG_EPI_STORE_PLAIN = 5,
  // kernel-internal: NLG_EPI_STORE_PLAIN that also records each wave's
  // start and end on the 100 MHz wall clock (FusedArgs::stamps)
  NLG_EPI_STORE_TIMED = 6,
};
struct FusedArgs {
  const float *x;        // [seq x cols] f32 activation rows
  const float *gain;     // PRO_RMS: [cols]
  float eps;             // PRO_RMS
  const uint32_t *w2;    // [out x wng] 2-bit rows
  const float *bias;     // [out] or null
  const float *beta;     // [1] or [out]
  int beta_per_row;
  uint32_t seq, out, cols, wng;
  float *y;              // output rows, ystride floats apart
  uint32_t ystride;
  const float *res;      // EPI_RESID, rstride floats apart (may equal y)
  uint32_t rstride;
  float *gamma_out;      // [seq] or null
  // EPI_QKV: q -> y; k, v -> caches [seq][kvheads][max_seq][hd] (fp16 bits)
  uint32_t nq, nkv, hd, kvheads, max_seq;
  // 0: row s is sequence s at position pos[0] (decode); else rows are
  // qper consecutive positions pos[0].. of each sequence (prefill)
  uint32_t qper;
  const float *co, *si;  // RoPE tables [max_seq x hd/2]
  const int32_t *pos;    // device position (one for every row of the batch)
  uint16_t *kc, *vc;
  // PRO_ATTN: x is [seq][attn_nc][cols] chunk contexts (a.x), with
  // (max, sum) per chunk and head in attn_mz [seq][attn_nc][cols/hd][2]
  const float *attn_mz;
  uint32_t attn_nc;
  // batched form: int8 activations + gamma ([seq x cols] bytes, then
  // [seq] floats at a 256-byte boundary); null = the library's scratch
  void *act_scratch;
  size_t act_scratch_bytes;
  // EPI_ARGMAX: per wave (max, index), [seq x ceil(out/R)]
  float *pval;
  int32_t *pidx;
  uint32_t nparts;
  // EPI_STORE_TIMED: [gridDim.x * 4 waves][2] (start, end) wall-clock stamps
  unsigned long long *stamps;
};
// Launch the fused kernel; rows_per_wave 0 picks a default.  Requires
// cols % 64 == 0, cols <= 16384 and 16-byte aligned x and w2.  With
// NLG_BATCHED_MIN or more tokens and cols % 256 == 0 it runs the batched
// form instead (per-token quantisation into library scratch, then the int8
// matrix-core GEMM with the same epilogue).
int nlg_fused_launch(const FusedArgs &a, int pro, int epi, int rows_per_wave, hipStream_t st);
// From 4 tokens the matrix-core form is faster than the decode GEMV, whose
// cost grows with every token (each workgroup quantises and dots one
// token; the quantise + GEMM pair is latency-bound and nearly flat).
// Measured on the config-4 FFN (2560 -> 6912 -> 2560): GEMV 14.3 / 16.4 /
// 19.3 / 27.1 / 31.7 us at 2 / 3 / 4 / 5 / 7 tokens, matrix cores 16.9 /
// 17.1 / 17.4 / 17.5 / 17.6 us; config-5 decode at batch 4 and 6: 3,079
// -> 3,202 and 3,617 -> 4,502 tok/s.
#define NLG_BATCHED_MIN 4
bool nlg_batched(uint32_t seq, uint32_t cols);
int nlg_batched_launch(const FusedArgs &a, int pro, int epi, hipStream_t st);
// Its GEMM alone, over activations already quantised into xq / gamma (as
// k_act_q leaves them); f's x, gain and prologue fields are not used.
int nlg_batched_gemm(const FusedArgs &f, const uint8_t *xq, const float *gamma, int epi, hipStream_t st);
// (max, index) partials per token an ARGMAX launch of `out` rows writes.
uint32_t nlg_argmax_parts(uint32_t seq, uint32_t cols, uint32_t out);
// Grow-only device scratch owned by the library, one per stream (NULL on
// failure).  It cannot grow while `st` is being captured into a graph.
void *nlg_scratch(size_t bytes, hipStream_t st);
// The same for another purpose (slot 1: zero-filled when allocated); NULL,
// with no error set, when it would have to grow inside a graph capture or
// cannot be allocated.
void *nlg_scratch_try(size_t bytes, hipStream_t st, int slot);
// The active device's fixed scratch array (NLG_NOALLOC_SCRATCH_BYTES), or
// null with the error set.
void *nlg_noalloc_scratch(void);
// The registered tiled copy of 2-bit weights w2 of rows x cols (the prefill
// GEMM's load order, nlg_repack.hip), or null; its size; and the release of
// every copy at shutdown.
const uint32_t *nlg_tiled_find(const uint32_t *w2, uint32_t rows, uint32_t cols);
size_t nlg_tiled_bytes(uint32_t rows, uint32_t cols);
void nlg_tiled_release_all(void);
// Refresh (in stream order) the copies of registrations overlapping a write
// of `bytes` at dst; drop those registered inside memory being freed.
void nlg_tiled_refresh_range(const void *dst, size_t bytes, hipStream_t st);
void nlg_tiled_drop_range(const void *base, size_t bytes);
// Bytes the batched form needs for seq tokens of cols columns.
size_t nlg_batched_scratch_bytes(uint32_t seq, uint32_t cols);
// The rows-per-wave the launcher uses for `out` rows in mode `epi`.
int nlg_fused_rows_per_wave(uint32_t out, int epi, uint32_t cols = 0);

// ---------------------------------------------------------------- launchers
// One per kernel name (Appendix A of the survey, lisp/nelisp-gpu-kernels.el).
#define NLG_DECL(fn) int fn(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st)
NLG_DECL(L_vadd);
NLG_DECL(L_add2);
NLG_DECL(L_mul);
NLG_DECL(L_scale);
NLG_DECL(L_causal_mask);
NLG_DECL(L_silu);
NLG_DECL(L_silu_mul);
NLG_DECL(L_rmsnorm_fwd);
NLG_DECL(L_embed_gather);
NLG_DECL(L_cache_append);
NLG_DECL(L_cache_append_b);
NLG_DECL(L_qkv_append);
NLG_DECL(L_decode_rope);
NLG_DECL(L_decode_rope_b);
NLG_DECL(L_rope_apply);
NLG_DECL(L_rope_half);
NLG_DECL(L_softmax);
NLG_DECL(L_rmsnorm_istd);
NLG_DECL(L_rmsnorm_heads);
NLG_DECL(L_pack_act_rows);
NLG_DECL(L_quant_act);
NLG_DECL(L_dp4a_dot);
NLG_DECL(L_bitlinear_dp4a);
NLG_DECL(L_bitlinear_dp4a_1f);
NLG_DECL(L_bitlinear_dp4a_rows);
NLG_DECL(L_ternary_rows);
NLG_DECL(L_bitlinear_packed);
NLG_DECL(L_bitlinear_packed_v);
NLG_DECL(L_matmul);
NLG_DECL(L_matmul_tiled);
NLG_DECL(L_matmul_reg);
NLG_DECL(L_linear);
NLG_DECL(L_attn_scores);
NLG_DECL(L_attn_context);
NLG_DECL(L_decode_attn);
NLG_DECL(L_decode_attn_b);
NLG_DECL(L_attn_causal_gqa);
NLG_DECL(L_ternary_i8);
NLG_DECL(L_decode_rope_b_v);
NLG_DECL(L_cache_append_ring);
NLG_DECL(L_cache_append_paged);
NLG_DECL(L_cache_append_paged_v);
NLG_DECL(L_block_copy);
NLG_DECL(L_decode_attn_stream);
NLG_DECL(L_attn_stream_entries);
NLG_DECL(L_decode_attn_paged);
NLG_DECL(L_decode_attn_paged_v);
NLG_DECL(L_ternary_rows_t);
NLG_DECL(L_dp4a_rows_t);
