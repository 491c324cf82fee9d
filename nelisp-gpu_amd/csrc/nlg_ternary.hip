// nlg_ternary.hip -- int8 activation quantisation and the ternary / int8
// linears: the decode GEMV at the centre of the hot path.
//
// Formats (lisp/nelisp-gpu-kernels.el):
//   activations  pack-act-rows (:884-932): per row gamma = amax/127 and four
//                signed int8 lanes per u32 word, lane l = column 4w+l.
//   2-bit weights ternary-rows (:700-746): 16 fields per u32, field f in bits
//                2f..2f+1, decoded by sign extension: 00 0, 01 +1, 11 -1, 10 -2.
//   int8 weights bitlinear-dp4a-1f (:619-634): four int8 lanes per u32.
//
// The 2-bit x int8 decode GEMV (nlg_ternary_linear_i8): a wave owns R output
// rows; each lane streams 16-byte chunks (4 words = 64 weights) of those rows
// with one global_load_dwordx4 per row, so a wave reads 1 KiB of contiguous
// row per instruction.  A field moved to bits 6..7 of its byte reads, as a
// signed int8, exactly 64x its decoded value (00->0, 01->64, 10->-128,
// 11->-64), so `(w << (6-2s)) & 0xC0C0C0C0` turns fields s, s+4, s+8, s+12
// of a word into a dot4 operand with no sign fix-up.  The matching
// activation bytes are gathered with v_perm_b32 (a 4x4 byte transpose per
// 16 columns, done once per wave and reused for every row).  The int32 sum
// is therefore 64x the exact accumulator and `>> 6` recovers it exactly;
// the fp32 epilogue is bitlinear-dp4a-1f's, evaluated without contraction.
#include "nlg_quant.h"

// ------------------------------------------------------------ quantisation

// One workgroup per row.  Pass 1: amax (order-free: the DSL max never
// selects a NaN and starts from 0).  Pass 2: one packed word per thread-step.
template <bool VEC4>
__global__ __launch_bounds__(256) void k_pack_act_rows(const float *__restrict__ x,
                                                       uint32_t *__restrict__ xq,
                                                       float *__restrict__ gamma, uint32_t rows,
                                                       uint32_t cols, uint32_t ng) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const float *xr = x + (size_t)row * cols;
  float amax = 0.0f;
  if (VEC4) {
    const float4 *x4 = (const float4 *)xr;
    for (uint32_t c = threadIdx.x; c < cols / 4; c += blockDim.x) {
      float4 v = x4[c];
      float a;
      a = dsl_abs(v.x); amax = a > amax ? a : amax;
      a = dsl_abs(v.y); amax = a > amax ? a : amax;
      a = dsl_abs(v.z); amax = a > amax ? a : amax;
      a = dsl_abs(v.w); amax = a > amax ? a : amax;
    }
  } else {
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
      float a = dsl_abs(xr[c]);
      amax = a > amax ? a : amax;
    }
  }
  amax = nlg_block_max_f32(amax, red);
  const float g = nlg_gamma_of(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(amax))));
  const float ginv = 1.0f / g;
  if (threadIdx.x == 0) gamma[row] = g;
  const bool fast = quant_fast(g);
  uint32_t *q = xq + (size_t)row * ng;
  for (uint32_t w = threadIdx.x; w < ng; w += blockDim.x) {
    uint32_t word = 0;
    if (VEC4 && 4 * w + 3 < cols) {
      word = quant_word(((const float4 *)xr)[w], g, ginv, fast);
    } else {
      for (uint32_t l = 0; l < 4; l++) {
        uint32_t c = 4 * w + l;
        if (c < cols) word |= pack_lane(xr[c], g) << (8 * l);
      }
    }
    q[w] = word;
  }
}

static int launch_pack_act(const float *x, uint32_t *xq, float *gamma, uint32_t rows, uint32_t cols,
                           uint32_t ng, hipStream_t st) {
  if (!rows) return NLG_OK;
  bool v4 = (cols % 4 == 0) && (((uintptr_t)x & 15) == 0);
  if (v4)
    hipLaunchKernelGGL(k_pack_act_rows<true>, dim3(rows), dim3(256), 0, st, x, xq, gamma, rows,
                       cols, ng);
  else
    hipLaunchKernelGGL(k_pack_act_rows<false>, dim3(rows), dim3(256), 0, st, x, xq, gamma, rows,
                       cols, ng);
  NLG_LAUNCHED("pack-act-rows");
  return NLG_OK;
}

extern "C" int nlg_pack_act_rows(const float *x, uint32_t *xq, float *gamma, uint32_t seq,
                                 uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  return launch_pack_act(x, xq, gamma, seq, cols, (cols + 3) / 4, nlg_stream(stream));
}

// pack-act-rows by name: X XQ GAMMA; push (seq cols ng)
int L_pack_act_rows(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], cols = p[1], ng = p[2];
  const uint64_t rows = nlg_domain(seq, groups);
  if (nlg_need(b, 0, rows * cols, "pack-act-rows") || nlg_need(b, 1, rows * ng, "pack-act-rows") ||
      nlg_need(b, 2, rows, "pack-act-rows"))
    return NLG_ERR;
  return launch_pack_act((const float *)b[0].ptr, (uint32_t *)b[1].ptr, (float *)b[2].ptr,
                         (uint32_t)rows, cols, ng, st);
}

// quant-act (kernels.el:527-547): fake quantisation, gamma*sgn*min(round,127).
__global__ __launch_bounds__(256) void k_quant_act(const float *__restrict__ x, float *__restrict__ xq,
                                                   uint32_t rows, uint32_t cols) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const float *xr = x + (size_t)row * cols;
  float amax = 0.0f;
  for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
    float a = dsl_abs(xr[c]);
    amax = a > amax ? a : amax;
  }
  amax = nlg_block_max_f32(amax, red);
  const float g = amax / 127.0f;
  __syncthreads();  // in place: every read of the row precedes any write
  for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
    float v = xr[c], out = 0.0f;
    if (g > 0.0f) {
      float q = v / g, sgn = 1.0f, aq = q;
      if (q < 0.0f) {
        sgn = -1.0f;
        aq = 0.0f - q;
      }
      uint32_t ri = nlg_f2u(aq + 0.5f);
      float rf = (float)ri;
      if (rf > 127.0f) rf = 127.0f;
      out = __fmul_rn(g, __fmul_rn(sgn, rf));
    }
    xq[(size_t)row * cols + c] = out;
  }
}

int L_quant_act(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], cols = p[1];
  const uint64_t rows = nlg_domain(seq, groups);
  if (nlg_need(b, 0, rows * cols, "quant-act") || nlg_need(b, 1, rows * cols, "quant-act"))
    return NLG_ERR;
  if (!rows) return NLG_OK;
  hipLaunchKernelGGL(k_quant_act, dim3((uint32_t)rows), dim3(256), 0, st, (const float *)b[0].ptr,
                     (float *)b[1].ptr, (uint32_t)rows, cols);
  NLG_LAUNCHED("quant-act");
  return NLG_OK;
}

// ------------------------------------------------------ 2-bit x int8 GEMV


struct TernArgs {
  const uint32_t *xq;    // [seq x ng]
  const float *gamma;    // [seq]
  const uint32_t *w2;    // [out x wng]
  const float *bias;     // [out] or null
  const float *beta;     // [1] or [out]
  float *y;              // [seq x out]
  uint32_t seq, out, cols, ng, wng;
  int beta_per_row;
  uint32_t wpb;          // waves per block (set by the launcher)
};

// Pin every argument into SGPRs at the top of a kernel: each kernel-argument
// fetch the compiler defers to first use is another memory round trip on the
// kernel's critical path.
#define TERN_PIN_ARGS(a)                                                                   \
  asm volatile("" ::"s"((a).xq), "s"((a).gamma), "s"((a).w2), "s"((a).bias), "s"((a).beta), \
               "s"((a).y), "s"((a).seq), "s"((a).out), "s"((a).cols), "s"((a).ng),          \
               "s"((a).wng), "s"((a).beta_per_row), "s"((a).wpb))

__device__ __forceinline__ void tern_store(const TernArgs &a, uint32_t s, uint32_t o, int acc64) {
  const float acc = (float)(acc64 >> 6);  // exact: acc64 is a multiple of 64
  const float bo = a.bias ? a.bias[o] : 0.0f;
  const float be = a.beta[a.beta_per_row ? o : 0];
  // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
  a.y[(size_t)s * a.out + o] = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, a.gamma[s]), acc));
}

// FAST path: cols % 64 == 0, so every row is a whole number of 16-byte
// chunks (4 words = 64 weights) and every activation row is 16-byte aligned.  R rows per wave, ST tokens per block
// (blockIdx.y picks the token tile).
template <int R, int ST>
__global__ __launch_bounds__(256) void k_tern_i8_fast(TernArgs a) {
  const int lane = threadIdx.x & 63;
  TERN_PIN_ARGS(a);
  const uint32_t wave = blockIdx.x * a.wpb + (threadIdx.x >> 6);
  const uint32_t row0 = wave * R;
  if (row0 >= a.out) return;  // wave-uniform
  const uint32_t s0 = blockIdx.y * ST;
  const uint32_t nchunk = a.wng >> 2;  // 4 words per chunk
  const uint4 *wrow[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    uint32_t row = row0 + r < a.out ? row0 + r : a.out - 1;  // tail rows: read a real row, discard
    wrow[r] = (const uint4 *)(a.w2 + (size_t)row * a.wng);
  }
  int acc[R][ST];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int s = 0; s < ST; s++) acc[r][s] = 0;
  // epilogue operands are loaded now, with the weights, not after the sums
  const uint32_t orow_u = row0 + (lane < R ? lane : 0);
  const uint32_t orow = orow_u < a.out ? orow_u : a.out - 1;  // every lane loads a valid row
  const bool olive = lane < R && orow_u < a.out;
  const float bo = a.bias ? a.bias[orow] : 0.0f;  // uniform test of a kernel argument
  const float be = a.beta[a.beta_per_row ? orow : 0];
  float gm[ST];
#pragma unroll
  for (int s = 0; s < ST; s++) gm[s] = (s0 + s < a.seq) ? a.gamma[s0 + s] : 0.0f;

  // Lanes leave this loop at different trips and reconverge after it, so the
  // DPP reductions below run with the full wave active.
  for (uint32_t c = lane; c < nchunk; c += 64) {
    const bool valid = true;
    uint4 wv[R];
#pragma unroll
    for (int r = 0; r < R; r++) wv[r] = nlg_ld_stream(&wrow[r][c]);
#pragma unroll
    for (int s = 0; s < ST; s++) {
      const uint32_t tok = s0 + s;
      if (ST > 1 && tok >= a.seq) break;
      uint4 xv[4];
      const uint4 *xr = (const uint4 *)(a.xq + (size_t)tok * a.ng) + 4 * c;
#pragma unroll
      for (int j = 0; j < 4; j++) xv[j] = valid ? xr[j] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        uint32_t y0, y1, y2, y3;
        xpose4(xv[j].x, xv[j].y, xv[j].z, xv[j].w, y0, y1, y2, y3);
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t w = j == 0 ? wv[r].x : j == 1 ? wv[r].y : j == 2 ? wv[r].z : wv[r].w;
          acc[r][s] = wdot(w, y0, y1, y2, y3, acc[r][s]);
        }
      }
    }
  }
#pragma unroll
  for (int s = 0; s < ST; s++) {
    const uint32_t tok = s0 + s;
    if (ST > 1 && tok >= a.seq) break;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int tot = nlg_wave_sum_i32(acc[r][s]);
      // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
      if (lane == r && olive)
        a.y[(size_t)tok * a.out + orow] = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, gm[s]), (float)(tot >> 6)));
    }
  }
}

// One token (the decode GEMV): cols % 64 == 0 and nchunk <= 64*CPL.  All of a
// lane's loads -- activation chunks (L2), weight chunks (HBM) and epilogue
// operands -- are issued as straight-line code before any use; invalid chunks
// read a clamped real address and are zeroed by selects, because a branch
// around a load makes the wait-count pass drain every load at the join.
template <int R, int CPL>
__global__ __launch_bounds__(256) void k_tern_i8_dec(TernArgs a) {
  const int lane = threadIdx.x & 63;
  TERN_PIN_ARGS(a);
  const uint32_t wave = blockIdx.x * a.wpb + (threadIdx.x >> 6);
  const uint32_t row0 = wave * R;
  if (row0 >= a.out) return;  // wave-uniform
  const uint32_t nchunk = a.wng >> 2;
  const uint32_t tok = blockIdx.y;
  uint4 xv[CPL][4];
  const uint4 *xr = (const uint4 *)(a.xq + (size_t)tok * a.ng);
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const uint32_t c = lane + 64u * i, cc = c < nchunk ? c : nchunk - 1;
#pragma unroll
    for (int j = 0; j < 4; j++) xv[i][j] = xr[4 * cc + j];
  }
  uint4 wv[R][CPL];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint32_t row = row0 + r < a.out ? row0 + r : a.out - 1;
    const uint4 *wr = (const uint4 *)(a.w2 + (size_t)row * a.wng);
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const uint32_t c = lane + 64u * i;
      wv[r][i] = nlg_ld_stream(&wr[c < nchunk ? c : nchunk - 1]);
    }
  }
  const uint32_t orow_u = row0 + (lane < R ? lane : 0);
  const uint32_t orow = orow_u < a.out ? orow_u : a.out - 1;
  const bool olive = lane < R && orow_u < a.out;
  const float *bsrc = a.bias ? a.bias : a.beta;
  const float bo_raw = bsrc[a.bias ? orow : 0];
  const float be = a.beta[a.beta_per_row ? orow : 0];
  const float gm = a.gamma[tok];
  const float bo = a.bias ? bo_raw : 0.0f;
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const bool valid = lane + 64u * i < nchunk;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t y0, y1, y2, y3;
      xpose4(xv[i][j].x, xv[i][j].y, xv[i][j].z, xv[i][j].w, y0, y1, y2, y3);
#pragma unroll
      for (int r = 0; r < R; r++) {
        uint32_t w = j == 0 ? wv[r][i].x : j == 1 ? wv[r][i].y : j == 2 ? wv[r][i].z : wv[r][i].w;
        w = valid ? w : 0u;
        acc[r] = wdot(w, y0, y1, y2, y3, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int tot = nlg_wave_sum_i32(acc[r]);
    // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
    if (lane == r && olive)
      a.y[(size_t)tok * a.out + orow] = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, gm), (float)(tot >> 6)));
  }
}

// GENERAL path: any cols.  One 2-bit word (16 columns) per lane-step, scalar
// loads; fields at or beyond `cols` are masked off and activation words past
// ng read as zero.
template <int R>
__global__ __launch_bounds__(256) void k_tern_i8_any(TernArgs a) {
  const int lane = threadIdx.x & 63;
  TERN_PIN_ARGS(a);
  const uint32_t wave = blockIdx.x * a.wpb + (threadIdx.x >> 6);
  const uint32_t row0 = wave * R;
  if (row0 >= a.out) return;
  const uint32_t tok = blockIdx.y;
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0;
  const uint32_t *xr = a.xq + (size_t)tok * a.ng;
  for (uint32_t j = lane; j < a.wng; j += 64) {
    const bool valid = true;
    uint32_t mask = 0xffffffffu;
    const uint32_t c0 = 16 * j;
    if (c0 + 16 > a.cols) mask = c0 >= a.cols ? 0u : ((1u << (2 * (a.cols - c0))) - 1u);
    uint32_t x4[4];
#pragma unroll
    for (int k = 0; k < 4; k++) x4[k] = (valid && 4 * j + k < a.ng) ? xr[4 * j + k] : 0u;
    uint32_t y0, y1, y2, y3;
    xpose4(x4[0], x4[1], x4[2], x4[3], y0, y1, y2, y3);
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r < a.out ? row0 + r : a.out - 1;
      const uint32_t w = valid ? (a.w2[(size_t)row * a.wng + j] & mask) : 0u;
      acc[r] = wdot(w, y0, y1, y2, y3, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int tot = nlg_wave_sum_i32(acc[r]);
    if (lane == r && row0 + r < a.out) tern_store(a, tok, row0 + r, tot);
  }
}

// Launch geometry.  rows_per_wave in {1,2,4,8}, waves_per_block in {1,2,4}.
static int tern_launch(const TernArgs &a0, int rows_per_wave, int waves_per_block, hipStream_t st) {
  TernArgs a = a0;
  a.wpb = (uint32_t)waves_per_block;
  if (!a.seq || !a.out) return NLG_OK;
  if (a.cols > 131072) return nlg_fail("ternary linear: cols %u > 131072", a.cols);
  const bool fast = (a.cols % 64 == 0) && (((uintptr_t)a.w2 & 15) == 0) &&
                    (((uintptr_t)a.xq & 15) == 0);
  const uint32_t threads = 64u * (uint32_t)waves_per_block;
  const uint64_t rows_per_block = (uint64_t)rows_per_wave * waves_per_block;
  dim3 blk(threads);
#define TERN_FAST(RR, SS)                                                                     \
  hipLaunchKernelGGL((k_tern_i8_fast<RR, SS>),                                               \
                     dim3(nlg_blocks(a.out, rows_per_block), (a.seq + SS - 1) / SS), blk, 0, st, a)
#define TERN_DEC(RR, CC) \
  hipLaunchKernelGGL((k_tern_i8_dec<RR, CC>), dim3(nlg_blocks(a.out, rows_per_block), 1), blk, 0, st, a)
#define TERN_FAST_R(RR)                                     \
  do {                                                      \
    if (a.seq == 1 && a.wng / 4 <= 64) TERN_DEC(RR, 1);     \
    else if (a.seq == 1 && a.wng / 4 <= 128) TERN_DEC(RR, 2); \
    else if (a.seq == 1) TERN_FAST(RR, 1);                  \
    else if (a.seq <= 2) TERN_FAST(RR, 2);                  \
    else if (a.seq <= 4) TERN_FAST(RR, 4);  \
    else TERN_FAST(RR, 8);                  \
  } while (0)
#define TERN_ANY(RR) \
  hipLaunchKernelGGL((k_tern_i8_any<RR>), dim3(nlg_blocks(a.out, rows_per_block), a.seq), blk, 0, st, a)
  if (fast) {
    switch (rows_per_wave) {
      case 1: TERN_FAST_R(1); break;
      case 2: TERN_FAST_R(2); break;
      case 8: TERN_FAST_R(8); break;
      default: TERN_FAST_R(4); break;
    }
  } else {
    switch (rows_per_wave) {
      case 1: TERN_ANY(1); break;
      case 2: TERN_ANY(2); break;
      case 8: TERN_ANY(8); break;
      default: TERN_ANY(4); break;
    }
  }
#undef TERN_FAST
#undef TERN_FAST_R
#undef TERN_DEC
#undef TERN_ANY
  NLG_LAUNCHED("ternary linear i8");
  return NLG_OK;
}

static void tern_default_geometry(uint32_t out, uint32_t seq, int *rpw, int *wpb) {
  // Enough waves to give every SIMD of 256 CUs work at decode shapes.
  (void)seq;
  *wpb = 4;
  // about two workgroups per CU measured best at 4096 rows (3.2 us)
  *rpw = out >= 2048 ? 2 : 1;
}

extern "C" int nlg_ternary_linear_i8_cfg(const uint32_t *xq, const float *gamma, const uint32_t *w2,
                                         const float *bias, const float *beta, int beta_per_row,
                                         float *y, uint32_t seq, uint32_t out, uint32_t cols,
                                         int rows_per_wave, int waves_per_block, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (rows_per_wave != 1 && rows_per_wave != 2 && rows_per_wave != 4 && rows_per_wave != 8)
    return nlg_fail("rows_per_wave must be 1, 2, 4 or 8");
  if (waves_per_block < 1 || waves_per_block > 4) return nlg_fail("waves_per_block must be 1..4");
  TernArgs a{xq, gamma, w2, bias, beta, y, seq, out, cols, (cols + 3) / 4, (cols + 15) / 16,
             beta_per_row};
  return tern_launch(a, rows_per_wave, waves_per_block, nlg_stream(stream));
}

extern "C" int nlg_ternary_linear_i8(const uint32_t *xq, const float *gamma, const uint32_t *w2,
                                     const float *bias, const float *beta, int beta_per_row,
                                     float *y, uint32_t seq, uint32_t out, uint32_t cols,
                                     void *stream) {
  int rpw, wpb;
  tern_default_geometry(out, seq, &rpw, &wpb);
  return nlg_ternary_linear_i8_cfg(xq, gamma, w2, bias, beta, beta_per_row, y, seq, out, cols, rpw,
                                   wpb, stream);
}

// ---------------------------------------- fused: quantise + GEMV, one launch
// (k_tern_fused in nlg_layer.hip; this entry point is its plain form)

// The three forms of the whole linear: one fused launch for a few tokens,
// the batched matrix-core form for many (its int8 activations in act_scratch,
// or the library's per-stream scratch when null), else pack-act-rows into
// the workspace and the GEMV.
static bool linear_fusable(const float *x, const uint32_t *w2, uint32_t seq, uint32_t cols) {
  const bool aligned = (((uintptr_t)x & 15) == 0) && (((uintptr_t)w2 & 15) == 0);
  return (cols % 64 == 0) && cols <= 16384 && aligned && (seq <= 4 || nlg_batched(seq, cols));
}

static int linear_go(const float *x, const uint32_t *w2, const float *bias, const float *beta, int beta_per_row,
                     float *y, float *gamma_out, uint32_t seq, uint32_t out, uint32_t cols, int rows_per_wave,
                     void *workspace, size_t workspace_bytes, void *act_scratch, size_t act_scratch_bytes,
                     hipStream_t st) {
  if (linear_fusable(x, w2, seq, cols)) {
    FusedArgs a{};
    a.x = x; a.w2 = w2; a.bias = bias; a.beta = beta; a.beta_per_row = beta_per_row;
    a.y = y; a.ystride = out; a.gamma_out = gamma_out; a.seq = seq; a.out = out; a.cols = cols;
    a.act_scratch = act_scratch; a.act_scratch_bytes = act_scratch_bytes;
    int rpw = rows_per_wave;
    if (rpw != 1 && rpw != 2 && rpw != 4) rpw = 0;  // the launcher's default
    return nlg_fused_launch(a, NLG_PRO_NONE, NLG_EPI_STORE, rpw, st);
  }
  // two launches: pack-act-rows into the workspace, then the GEMV
  const size_t ng = (cols + 3) / 4;
  const size_t need = (seq * ng * 4 + 255) / 256 * 256 + (size_t)seq * 4;
  if (!workspace || workspace_bytes < need)
    return nlg_fail("ternary linear: this shape needs a %zu-byte workspace", need);
  uint32_t *xq = (uint32_t *)workspace;
  float *gm = gamma_out ? gamma_out : (float *)((char *)workspace + (seq * ng * 4 + 255) / 256 * 256);
  if (launch_pack_act(x, xq, gm, seq, cols, (uint32_t)ng, st)) return NLG_ERR;
  TernArgs ta{xq, gm, w2, bias, beta, y, seq, out, cols, (uint32_t)ng, (cols + 15) / 16, beta_per_row};
  int rpw, wpb;
  tern_default_geometry(out, seq, &rpw, &wpb);
  return tern_launch(ta, rpw, wpb, st);
}

// The bare one-token linear (no bias, one beta, no gamma output) with each
// wave's start and end stamped on the device's 100 MHz wall clock: a
// device-side duration of graph-replayed launches, no profiler attached.
extern "C" int nlg_ternary_linear_timed(const float *x, const uint32_t *w2, const float *beta, float *y,
                                        uint32_t out, uint32_t cols, unsigned long long *stamps,
                                        size_t stamps_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!out) return NLG_OK;
  if (!x || !w2 || !beta || !y || !stamps) return nlg_fail("timed linear: null pointer");
  if (!linear_fusable(x, w2, 1, cols)) return nlg_fail("timed linear: cols must be a multiple of 64 in [64, 16384]");
  if (stamps_bytes < nlg_ternary_linear_timed_stamps(out)) return nlg_fail("timed linear: stamps buffer is short");
  FusedArgs a{};
  a.x = x; a.w2 = w2; a.beta = beta; a.y = y; a.ystride = out; a.seq = 1; a.out = out; a.cols = cols;
  a.stamps = stamps;
  return nlg_fused_launch(a, NLG_PRO_NONE, NLG_EPI_STORE, 0, nlg_stream(stream));
}

// 16 bytes per wave of the default geometry (4 waves per workgroup)
extern "C" size_t nlg_ternary_linear_timed_stamps(uint32_t out) {
  const uint32_t rpw = (uint32_t)nlg_fused_rows_per_wave(out, NLG_EPI_STORE);
  return (size_t)((out + 4 * rpw - 1) / (4 * rpw)) * 4 * 16;
}

extern "C" int nlg_ternary_linear_cfg(const float *x, const uint32_t *w2, const float *bias,
                                      const float *beta, int beta_per_row, float *y, float *gamma_out,
                                      uint32_t seq, uint32_t out, uint32_t cols, int rows_per_wave,
                                      void *workspace, size_t workspace_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!seq || !out) return NLG_OK;
  return linear_go(x, w2, bias, beta, beta_per_row, y, gamma_out, seq, out, cols, rows_per_wave, workspace,
                   workspace_bytes, nullptr, 0, nlg_stream(stream));
}

// The same linear with every scratch byte in the library's fixed array:
// no allocation on any path (for graph capture and callers that cannot
// allocate).  Calls that overlap on one GPU share the array and race.
extern "C" int nlg_ternary_linear_noalloc(const float *x, const uint32_t *w2, const float *bias,
                                          const float *beta, int beta_per_row, float *y, float *gamma_out,
                                          uint32_t seq, uint32_t out, uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!seq || !out) return NLG_OK;
  const size_t need = linear_fusable(x, w2, seq, cols)
                          ? (nlg_batched(seq, cols) ? nlg_batched_scratch_bytes(seq, cols) : 0)
                          : nlg_ternary_linear_workspace(seq, cols);
  if (need > NLG_NOALLOC_SCRATCH_BYTES)
    return nlg_fail("ternary linear (no allocation): %u tokens x %u columns need %zu bytes of scratch, "
                    "more than the fixed %zu", seq, cols, need, (size_t)NLG_NOALLOC_SCRATCH_BYTES);
  void *scr = nlg_noalloc_scratch();
  if (!scr) return NLG_ERR;
  return linear_go(x, w2, bias, beta, beta_per_row, y, gamma_out, seq, out, cols, 0, scr,
                   NLG_NOALLOC_SCRATCH_BYTES, scr, NLG_NOALLOC_SCRATCH_BYTES, nlg_stream(stream));
}

extern "C" size_t nlg_ternary_linear_workspace(uint32_t seq, uint32_t cols) {
  const size_t ng = (cols + 3) / 4;
  return (seq * ng * 4 + 255) / 256 * 256 + (size_t)seq * 4;
}

extern "C" int nlg_ternary_linear(const float *x, const uint32_t *w2, const float *bias,
                                  const float *beta, int beta_per_row, float *y, float *gamma_out,
                                  uint32_t seq, uint32_t out, uint32_t cols, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  return nlg_ternary_linear_cfg(x, w2, bias, beta, beta_per_row, y, gamma_out, seq, out, cols, 0,
                                workspace, workspace_bytes, stream);
}

// "ternary-i8" by name (an extension with no reference counterpart: the
// composite the reference expresses as pack-act-rows + bitlinear-dp4a-1f on
// unpacked weights).  AP WP BIAS BETA GAMMA Y; push (seq out cols).  One
// invocation per output, idx = s*out + o < min(seq*out, 64*groups): a partial
// grid is the whole rows s < n/out, then the first n%out outputs of row n/out.
int L_ternary_i8(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], out = p[1], cols = p[2];
  const uint32_t ng = (cols + 3) / 4, wng = (cols + 15) / 16;
  const char *k = "ternary-i8";
  if (nlg_need(b, 0, (uint64_t)seq * ng, k) || nlg_need(b, 1, (uint64_t)out * wng, k) ||
      nlg_need(b, 2, out, k) || nlg_need(b, 3, 1, k) || nlg_need(b, 4, seq, k) ||
      nlg_need(b, 5, (uint64_t)seq * out, k))
    return NLG_ERR;
  if (!seq || !out) return NLG_OK;
  const uint64_t n = nlg_domain((uint64_t)seq * out, groups);
  const uint32_t full = (uint32_t)(n / out), part = (uint32_t)(n % out);
  const uint32_t *xq = (const uint32_t *)b[0].ptr;
  const float *gamma = (const float *)b[4].ptr;
  float *y = (float *)b[5].ptr;
  int rpw, wpb;
  if (full) {
    TernArgs a{xq, gamma, (const uint32_t *)b[1].ptr, (const float *)b[2].ptr, (const float *)b[3].ptr, y, full,
               out, cols, ng, wng, 0};
    tern_default_geometry(out, full, &rpw, &wpb);
    if (tern_launch(a, rpw, wpb, st)) return NLG_ERR;
  }
  if (part) {  // row `full`, outputs 0..part-1
    TernArgs a{xq + (size_t)full * ng, gamma + full, (const uint32_t *)b[1].ptr, (const float *)b[2].ptr,
               (const float *)b[3].ptr, y + (size_t)full * out, 1, part, cols, ng, wng, 0};
    tern_default_geometry(part, 1, &rpw, &wpb);
    if (tern_launch(a, rpw, wpb, st)) return NLG_ERR;
  }
  return NLG_OK;
}

// ------------------------------------------------------ int8-lane linears

// bitlinear-dp4a-1f / -rows / bitlinear-dp4a: one wave per output (s, o),
// lanes stride over the ng words; int32 sums are exact in any order.
// CARRY: words arrive as two f32 halves lo + hi*65536 (bitlinear-dp4a).
template <bool CARRY>
__global__ __launch_bounds__(256) void k_dp4a_rows(const float *ap, const float *ahi, const float *wp,
                                                   const float *whi, const float *bias, const float *beta,
                                                   const float *gamma, float *y, uint32_t n_out,
                                                   uint32_t out, uint32_t ng, int per_row) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wave >= n_out) return;
  const uint32_t idx = (uint32_t)wave, s = idx / out, o = idx % out;
  const uint32_t ab = s * ng, wb = o * ng;
  int acc = 0;
  for (uint32_t g = lane; g < ((ng + 63) & ~63u); g += 64) {
    if (g < ng) {
      uint32_t a_, w_;
      if (CARRY) {
        a_ = nlg_f2u(ap[ab + g]) + nlg_f2u(ahi[ab + g]) * 65536u;
        w_ = nlg_f2u(wp[wb + g]) + nlg_f2u(whi[wb + g]) * 65536u;
      } else {
        a_ = __float_as_uint(ap[ab + g]);
        w_ = __float_as_uint(wp[wb + g]);
      }
      acc = __builtin_amdgcn_sdot4((int)a_, (int)w_, acc, false);
    }
  }
  acc = nlg_wave_sum_i32(acc);
  if (lane == 0)
    y[idx] = __fadd_rn(bias[o], __fmul_rn(__fmul_rn(beta[per_row ? o : 0], gamma[s]), (float)acc));
}

static int dp4a_common(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st,
                       bool carry, int per_row, const char *k) {
  const uint32_t seq = p[0], out = p[1], ng = p[2];
  const uint64_t n = nlg_domain((uint64_t)seq * out, groups);
  if (!n) return NLG_OK;
  const uint64_t srows = (n + out - 1) / out;  // tokens touched
  const int ia = 0, iw = carry ? 2 : 1, ib = carry ? 4 : 2, ibe = carry ? 5 : 3,
            ig = carry ? 6 : 4, iy = carry ? 7 : 5;
  if (nlg_need(b, ia, srows * ng, k) || nlg_need(b, iw, (uint64_t)out * ng, k) ||
      nlg_need(b, ib, out, k) || nlg_need(b, ibe, per_row ? out : 1, k) ||
      nlg_need(b, ig, srows, k) || nlg_need(b, iy, n, k))
    return NLG_ERR;
  if (carry && (nlg_need(b, 1, srows * ng, k) || nlg_need(b, 3, (uint64_t)out * ng, k)))
    return NLG_ERR;
  const float *a0 = (const float *)b[ia].ptr, *w0 = (const float *)b[iw].ptr;
  const float *a1 = carry ? (const float *)b[1].ptr : nullptr;
  const float *w1 = carry ? (const float *)b[3].ptr : nullptr;
  if (carry)
    hipLaunchKernelGGL(k_dp4a_rows<true>, dim3(nlg_blocks(n, 4)), dim3(256), 0, st, a0, a1, w0, w1,
                       (const float *)b[ib].ptr, (const float *)b[ibe].ptr,
                       (const float *)b[ig].ptr, (float *)b[iy].ptr, (uint32_t)n, out, ng, per_row);
  else
    hipLaunchKernelGGL(k_dp4a_rows<false>, dim3(nlg_blocks(n, 4)), dim3(256), 0, st, a0, a1, w0, w1,
                       (const float *)b[ib].ptr, (const float *)b[ibe].ptr,
                       (const float *)b[ig].ptr, (float *)b[iy].ptr, (uint32_t)n, out, ng, per_row);
  NLG_LAUNCHED(k);
  return NLG_OK;
}

int L_bitlinear_dp4a_1f(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return dp4a_common(b, p, groups, st, false, 0, "bitlinear-dp4a-1f");
}
int L_bitlinear_dp4a_rows(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return dp4a_common(b, p, groups, st, false, 1, "bitlinear-dp4a-rows");
}
int L_bitlinear_dp4a(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return dp4a_common(b, p, groups, st, true, 0, "bitlinear-dp4a");
}

// dp4a-dot (kernels.el:587-600)
__global__ void k_dp4a_dot(const float *alo, const float *ahi, const float *blo, const float *bhi,
                           float *out, uint32_t n) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    uint32_t a = nlg_f2u(alo[i]) + nlg_f2u(ahi[i]) * 65536u;
    uint32_t c = nlg_f2u(blo[i]) + nlg_f2u(bhi[i]) * 65536u;
    out[i] = (float)__builtin_amdgcn_sdot4((int)a, (int)c, 0, false);
  }
}
int L_dp4a_dot(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint64_t n = nlg_domain(p[0], groups);
  for (int i = 0; i < 5; i++)
    if (nlg_need(b, i, n, "dp4a-dot")) return NLG_ERR;
  if (!n) return NLG_OK;
  hipLaunchKernelGGL(k_dp4a_dot, dim3(nlg_blocks(n, 256)), dim3(256), 0, st, (const float *)b[0].ptr,
                     (const float *)b[1].ptr, (const float *)b[2].ptr, (const float *)b[3].ptr,
                     (float *)b[4].ptr, (uint32_t)n);
  NLG_LAUNCHED("dp4a-dot");
  return NLG_OK;
}

// ------------------------------------------------------ f32-activation linears

// ternary-rows (kernels.el:700-746): f32 activations, 2-bit weights, one
// scale per 128-column block.  One wave per output; lane-partial sums are
// scaled per word by the word's block beta (reassociated: tolerance parity).
__global__ __launch_bounds__(256) void k_ternary_rows(const float *x, const uint32_t *wp,
                                                      const float *bias, const float *beta, float *y,
                                                      uint32_t n_out, uint32_t out, uint32_t cols,
                                                      uint32_t nblk, uint32_t wng) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wave >= n_out) return;
  const uint32_t idx = (uint32_t)wave, s = idx / out, o = idx % out;
  const float *xr = x + (size_t)s * cols;
  const uint32_t *wr = wp + (size_t)o * wng;
  // the reference visits words wi = b*8 + w < wng for b < nblk only
  const uint32_t nw = wng < 8u * nblk ? wng : 8u * nblk;
  float acc = 0.0f;
  for (uint32_t wi = lane; wi < ((nw + 63) & ~63u); wi += 64) {
    if (wi < nw) {
      const uint32_t w = wr[wi];
      float part = 0.0f;
#pragma unroll
      for (uint32_t f = 0; f < 16; f++) {
        const uint32_t i = wi * 16 + f;
        if (i < cols) {
          const float sv = (float)((int32_t)(w << (30 - 2 * f)) >> 30);
          part = __fadd_rn(part, __fmul_rn(sv, xr[i]));
        }
      }
      acc = __fadd_rn(acc, __fmul_rn(beta[(size_t)o * nblk + wi / 8], part));
    }
  }
  acc = nlg_wave_sum_f32(acc);
  if (lane == 0) y[idx] = __fadd_rn(bias[o], acc);
}

int L_ternary_rows(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], out = p[1], cols = p[2], nblk = p[3], wng = p[4];
  const uint64_t n = nlg_domain((uint64_t)seq * out, groups);
  if (!n) return NLG_OK;
  const uint64_t srows = (n + out - 1) / out;
  const uint32_t nw = wng < 8u * nblk ? wng : 8u * nblk;
  const char *k = "ternary-rows";
  uint64_t xneed = srows ? (srows - 1) * cols + (uint64_t)(nw * 16 < cols ? nw * 16 : cols) : 0;
  if (nlg_need(b, 0, xneed, k) || nlg_need(b, 1, (uint64_t)(out - 1) * wng + nw, k) ||
      nlg_need(b, 2, out, k) || nlg_need(b, 3, (uint64_t)out * nblk, k) || nlg_need(b, 4, n, k))
    return NLG_ERR;
  hipLaunchKernelGGL(k_ternary_rows, dim3(nlg_blocks(n, 4)), dim3(256), 0, st,
                     (const float *)b[0].ptr, (const uint32_t *)b[1].ptr, (const float *)b[2].ptr,
                     (const float *)b[3].ptr, (float *)b[4].ptr, (uint32_t)n, out, cols, nblk, wng);
  NLG_LAUNCHED(k);
  return NLG_OK;
}

// bitlinear-packed / -v (kernels.el:992-1040): base-4 codes tern+1, pk per
// f32 value read with (uint f).  One wave per output.
__global__ __launch_bounds__(256) void k_bitlinear_packed(const float *x, const float *wpk,
                                                          const float *bias, const float *beta,
                                                          float *y, uint32_t n_out, uint32_t in,
                                                          uint32_t out, uint32_t pk, uint32_t fcount,
                                                          int per_row) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wave >= n_out) return;
  const uint32_t idx = (uint32_t)wave, s = idx / out, o = idx % out;
  const float be = beta[per_row ? o : 0];
  const float *xr = x + (size_t)s * in;
  const float *wr = wpk + (size_t)o * fcount;
  float acc = 0.0f;
  for (uint32_t f = lane; f < ((fcount + 63) & ~63u); f += 64) {
    if (f < fcount) {
      uint32_t packed = nlg_f2u(wr[f]);
      const uint32_t i0 = f * pk;
      for (uint32_t z = 0; z < pk; z++) {
        const uint32_t i = i0 + z;
        if (i < in) {
          const float tern = __fsub_rn((float)(packed % 4u), 1.0f);
          acc = __fadd_rn(acc, __fmul_rn(xr[i], __fmul_rn(be, tern)));
        }
        packed = packed / 4u;
      }
    }
  }
  acc = nlg_wave_sum_f32(acc);
  if (lane == 0) y[idx] = __fadd_rn(bias[o], acc);
}

static int packed_common(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st,
                         int per_row, const char *k) {
  const uint32_t seq = p[0], in = p[1], out = p[2], pk = p[3], fcount = p[4];
  const uint64_t n = nlg_domain((uint64_t)seq * out, groups);
  if (!n) return NLG_OK;
  const uint64_t srows = (n + out - 1) / out;
  uint64_t used = (uint64_t)fcount * pk < in ? (uint64_t)fcount * pk : in;
  if (nlg_need(b, 0, srows ? (srows - 1) * in + used : 0, k) ||
      nlg_need(b, 1, (uint64_t)out * fcount, k) || nlg_need(b, 2, out, k) ||
      nlg_need(b, 3, per_row ? out : 1, k) || nlg_need(b, 4, n, k))
    return NLG_ERR;
  hipLaunchKernelGGL(k_bitlinear_packed, dim3(nlg_blocks(n, 4)), dim3(256), 0, st,
                     (const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr,
                     (const float *)b[3].ptr, (float *)b[4].ptr, (uint32_t)n, in, out, pk, fcount,
                     per_row);
  NLG_LAUNCHED(k);
  return NLG_OK;
}
int L_bitlinear_packed(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return packed_common(b, p, groups, st, 0, "bitlinear-packed");
}
int L_bitlinear_packed_v(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return packed_common(b, p, groups, st, 1, "bitlinear-packed-v");
}
