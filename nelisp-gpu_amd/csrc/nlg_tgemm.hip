// nlg_tgemm.hip -- the batched (prefill / multi-sequence decode) form of the
// ternary linears: int8 activations x 2-bit weights on the int8 matrix cores.
//
// k_act_q: one workgroup per token row: optional RMSNorm (rmsnorm-istd +
// rmsnorm-fwd, kernels.el:1249-1265) or attention-chunk merge, then
// pack-act-rows' quantisation (kernels.el:884-932, exact; see nlg_quant.h)
// into the layout the GEMM's A operand reads: for every 16-column group the
// 16 int8 lanes in the order 0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15 (the
// 4x4 byte transpose of pack-act-rows' words), plus gamma per token.
//
// k_tgemm: Y[s, o] = epilogue(sum_c int8(x[s, c]) * decode(W[o, c])) with
// v_mfma_i32_16x16x64_i8.  A workgroup owns 64 output rows (16 per wave) and
// MT tokens; it walks the columns in chunks of 256 (16 2-bit words per row).
// Each lane fetches one 16-byte chunk of its weight row straight from HBM
// into registers and decodes it there: a field moved to bits 6..7 of a byte
// is 64x its value as a signed int8, so `(w << (6-2s)) & 0xC0C0C0C0` gives
// the B operand for columns 16w + 4b + s -- the order k_act_q stores A in.
// The int32 sum is 64x the exact accumulator (>> 6 recovers it); it is the
// same integer as bitlinear-dp4a-1f's (kernels.el:619-634), so every
// epilogue below produces the same bits as the GEMV kernels.
//
// Matrix-core operand layout (v_mfma_i32_16x16x64_i8, checked on gfx950):
// C[i][j] = sum over lane groups g = 0..3 and bytes b = 0..15 of
// A[lane 16g + i][b] * B[lane 16g + j][b], and lane l's result r is
// C[4(l/16) + r][l % 16].  Here i = token, j = output row, and lane group g
// at step t of a chunk covers 2-bit word 4g + t of the chunk.
#include <math.h>

#include "nlg_quant.h"

typedef int v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ k_act_q

struct ActQArgs {
  const float *x;       // [seq x cols] (PRO_NONE / PRO_RMS) or attention partials (PRO_ATTN)
  const float *gain;    // PRO_RMS
  float eps;
  const float *attn_mz; // PRO_ATTN: [seq][nc][heads][2]
  uint32_t attn_nc, hd;
  uint8_t *xq;          // [seq x cols] int8 in MFMA order
  float *gamma;         // [seq]
  uint32_t seq, cols;
};

// G16: 16-column groups per thread (cols <= 4096 * G16).
template <int G16, int PRO>
__global__ __launch_bounds__(256) void k_act_q(ActQArgs a) {
  __shared__ float red[4];
  asm volatile("" ::"s"(a.x), "s"(a.gain), "s"(a.xq), "s"(a.gamma), "s"(a.cols));
  const uint32_t tok = blockIdx.x;
  const uint32_t ngrp = a.cols >> 4, nf4 = a.cols >> 2;
  float4 v[G16][4];
  if (PRO == NLG_PRO_ATTN) {
    // attention merged from its chunks, in k_attn_merge's operation order
    const uint32_t heads = a.cols / a.hd;
    const float4 *c4 = (const float4 *)a.x;
#pragma unroll
    for (int k = 0; k < G16; k++) {
      const uint32_t gi = threadIdx.x + 256u * k, gc = gi < ngrp ? gi : ngrp - 1;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t f = 4 * gc + q, h = (4 * f) / a.hd;
        float4 cx[NLG_ATTN_MAX_CHUNKS];
        float2 mz[NLG_ATTN_MAX_CHUNKS];
#pragma unroll
        for (int c = 0; c < NLG_ATTN_MAX_CHUNKS; c++) {
          const uint32_t cc = (uint32_t)c < a.attn_nc ? (uint32_t)c : a.attn_nc - 1;
          const size_t tc = (size_t)tok * a.attn_nc + cc;
          cx[c] = c4[tc * nf4 + f];
          mz[c] = *(const float2 *)(a.attn_mz + (tc * heads + h) * 2);
        }
        float mm = -1.0e30f;
#pragma unroll
        for (int c = 0; c < NLG_ATTN_MAX_CHUNKS; c++) mm = mz[c].x > mm ? mz[c].x : mm;
        float zz = 0.0f;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int c = 0; c < NLG_ATTN_MAX_CHUNKS; c++) {
          const float sc = (uint32_t)c < a.attn_nc ? expf(mz[c].x - mm) : 0.0f;
          zz = fmaf(mz[c].y, sc, zz);
          acc.x = fmaf(cx[c].x, sc, acc.x);
          acc.y = fmaf(cx[c].y, sc, acc.y);
          acc.z = fmaf(cx[c].z, sc, acc.z);
          acc.w = fmaf(cx[c].w, sc, acc.w);
        }
        v[k][q] = make_float4(acc.x / zz, acc.y / zz, acc.z / zz, acc.w / zz);
      }
    }
  } else {
    const float4 *x4 = (const float4 *)(a.x + (size_t)tok * a.cols);
#pragma unroll
    for (int k = 0; k < G16; k++) {
      const uint32_t gi = threadIdx.x + 256u * k, gc = gi < ngrp ? gi : ngrp - 1;
#pragma unroll
      for (int q = 0; q < 4; q++) v[k][q] = x4[4 * gc + q];
    }
  }
  float4 gv[G16][4];
  if (PRO == NLG_PRO_RMS) {
    const float4 *g4 = (const float4 *)a.gain;
#pragma unroll
    for (int k = 0; k < G16; k++) {
      const uint32_t gi = threadIdx.x + 256u * k, gc = gi < ngrp ? gi : ngrp - 1;
#pragma unroll
      for (int q = 0; q < 4; q++) gv[k][q] = g4[4 * gc + q];
    }
  }
#pragma unroll
  for (int k = 0; k < G16; k++)
    if (threadIdx.x + 256u * k >= ngrp)
#pragma unroll
      for (int q = 0; q < 4; q++) v[k][q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (PRO == NLG_PRO_RMS) {
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < G16; k++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        sq = sq + v[k][q].x * v[k][q].x;
        sq = sq + v[k][q].y * v[k][q].y;
        sq = sq + v[k][q].z * v[k][q].z;
        sq = sq + v[k][q].w * v[k][q].w;
      }
    sq = nlg_block_sum_f32<4>(sq, red);
    sq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq)));
    const float istd = 1.0f / sqrtf(sq / (float)a.cols + a.eps);
#pragma unroll
    for (int k = 0; k < G16; k++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        v[k][q].x = (v[k][q].x * istd) * gv[k][q].x;
        v[k][q].y = (v[k][q].y * istd) * gv[k][q].y;
        v[k][q].z = (v[k][q].z * istd) * gv[k][q].z;
        v[k][q].w = (v[k][q].w * istd) * gv[k][q].w;
      }
  }
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < G16; k++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float t;
      t = dsl_abs(v[k][q].x); amax = t > amax ? t : amax;
      t = dsl_abs(v[k][q].y); amax = t > amax ? t : amax;
      t = dsl_abs(v[k][q].z); amax = t > amax ? t : amax;
      t = dsl_abs(v[k][q].w); amax = t > amax ? t : amax;
    }
  amax = nlg_block_max_f32<4>(amax, red);
  const float g = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(amax))) / 127.0f;
  const float ginv = 1.0f / g;
  const bool fast = g > 0.0f && ginv < INFINITY;
  if (threadIdx.x == 0) a.gamma[tok] = g;
  uint4 *dst = (uint4 *)(a.xq + (size_t)tok * a.cols);
#pragma unroll
  for (int k = 0; k < G16; k++) {
    const uint32_t gi = threadIdx.x + 256u * k;
    const uint32_t n0 = quant_word(v[k][0], g, ginv, fast), n1 = quant_word(v[k][1], g, ginv, fast);
    const uint32_t n2 = quant_word(v[k][2], g, ginv, fast), n3 = quant_word(v[k][3], g, ginv, fast);
    uint32_t y0, y1, y2, y3;
    xpose4(n0, n1, n2, n3, y0, y1, y2, y3);
    if (gi < ngrp) dst[gi] = make_uint4(y0, y1, y2, y3);
  }
}

// ------------------------------------------------------------ k_tgemm

struct GemmArgs {
  const uint8_t *xq;   // [seq x cols] MFMA-ordered int8 (k_act_q)
  const float *gamma;  // [seq]
  const uint32_t *w2;  // [out x wng]
  const float *bias;   // [out] or null
  const float *beta;   // [1] or [out]
  int beta_per_row;
  uint32_t seq, out, cols, wng;
  float *y;
  uint32_t ystride;
  const float *res;
  uint32_t rstride;
  // EPI_QKV
  uint32_t nq, nkv, hd, kvheads, max_seq;
  const float *co, *si;
  const int32_t *pos;
  uint16_t *kc, *vc;
  uint32_t qper;       // QKV: 0 = token s is sequence s at pos[0]; else sequence s/qper at pos[0] + s%qper
  // EPI_ARGMAX: per (token, workgroup) max and first index
  float *pval;
  int32_t *pidx;
  uint32_t nparts;
};

#define TG_KC 256                 // columns per chunk (16 2-bit words of a row)
#define TG_PH 8                   // chunks per phase
#define TG_PITCH (TG_PH * TG_KC + 16)  // LDS row pitch in bytes (staggers the banks)

// MB: 16-token blocks per workgroup (MT = 16*MB tokens).  The columns go in
// phases of 8 chunks (2048 columns): at the start of a phase every lane issues
// the loads of its weight row's 8 chunks (registers) and the workgroup's
// MT x 2048 activation block (to LDS), so a phase costs one memory round
// trip; then 8 x 4 x MB matrix-core steps run out of registers and LDS.
// NPH: phases (compile-time, so the loop over them unrolls and the staging
// arrays stay in registers): cols <= 2048 * NPH.
template <int MB, int NPH, int EPI>
__global__ __launch_bounds__(256) void k_tgemm(GemmArgs a) {
  constexpr int MT = 16 * MB;
  extern __shared__ __align__(16) uint8_t s_a[];  // MT x TG_PITCH
  __shared__ float s_bv[4][MT];
  __shared__ int32_t s_bi[4][MT];
  asm volatile("" ::"s"(a.xq), "s"(a.gamma), "s"(a.w2), "s"(a.bias), "s"(a.beta), "s"(a.y), "s"(a.seq),
               "s"(a.out), "s"(a.cols), "s"(a.wng), "s"(a.ystride), "s"(a.beta_per_row));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t row = blockIdx.x * 64 + w * 16 + lr;  // this lane's output row (B column j)
  const uint32_t rowc = row < a.out ? row : a.out - 1;
  const uint32_t tok0 = blockIdx.y * MT;
  const uint32_t nchunks = a.cols / TG_KC;
  const uint4 *wrow = (const uint4 *)(a.w2 + (size_t)rowc * a.wng);
  // activation staging: piece p = threadIdx.x + 256 i is token p / 128,
  // 16-byte slot p % 128 of the phase's 2048 columns
  constexpr int NA = MT * (TG_PH * TG_KC / 16) / 256;  // pieces per thread (8 MB)
  const uint32_t slot = threadIdx.x % 128u, tsub = threadIdx.x / 128u;  // token = tsub + 2i
  const float bo_raw = (a.bias ? a.bias : a.beta)[a.bias ? rowc : 0];
  const float be = a.beta[a.beta_per_row ? rowc : 0];
  const float bo = a.bias ? bo_raw : 0.0f;
  v4i acc[MB];
#pragma unroll
  for (int m = 0; m < MB; m++) acc[m] = (v4i){0, 0, 0, 0};
  // The staging registers are ext_vector values indexed by constants, not
  // arrays: an array here ends up in scratch once the phase loop unrolls.
  typedef uint32_t wvec_t __attribute__((ext_vector_type(4 * TG_PH)));
  typedef uint32_t avec_t __attribute__((ext_vector_type(4 * NA)));
#pragma unroll
  for (int ph = 0; ph < NPH; ph++) {
    const uint32_t c0 = ph * TG_PH;
    if (c0 >= nchunks) break;  // uniform
    wvec_t wv;
#pragma unroll
    for (int i = 0; i < TG_PH; i++) {
      const uint32_t cc = c0 + i < nchunks ? c0 + i : nchunks - 1;
      const uint4 u = wrow[4 * cc + lg];
      // chunks past the end contribute zero
      const uint32_t keep = c0 + i < nchunks ? 0xffffffffu : 0u;
      wv[4 * i + 0] = u.x & keep;
      wv[4 * i + 1] = u.y & keep;
      wv[4 * i + 2] = u.z & keep;
      wv[4 * i + 3] = u.w & keep;
    }
    avec_t ar;
    const uint32_t col = c0 * TG_KC + 16 * slot;
    const uint32_t colc = col < a.cols ? col : a.cols - 16;
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const uint32_t t = tsub + 2 * i, tk = tok0 + t < a.seq ? tok0 + t : a.seq - 1;
      const uint4 u = *(const uint4 *)(a.xq + (size_t)tk * a.cols + colc);
      ar[4 * i + 0] = u.x;
      ar[4 * i + 1] = u.y;
      ar[4 * i + 2] = u.z;
      ar[4 * i + 3] = u.w;
    }
    if (c0) __syncthreads();  // every wave is done with the previous phase's block
#pragma unroll
    for (int i = 0; i < NA; i++)
      *(uint4 *)(&s_a[(tsub + 2 * i) * TG_PITCH + 16 * slot]) =
          make_uint4(ar[4 * i], ar[4 * i + 1], ar[4 * i + 2], ar[4 * i + 3]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TG_PH; i++) {
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t wd = wv[4 * i + t];
        const v4i bop = {(int)((wd << 6) & 0xC0C0C0C0u), (int)((wd << 4) & 0xC0C0C0C0u),
                         (int)((wd << 2) & 0xC0C0C0C0u), (int)(wd & 0xC0C0C0C0u)};
#pragma unroll
        for (int m = 0; m < MB; m++) {
          const uint4 av = *(const uint4 *)(s_a + (16 * m + lr) * TG_PITCH + i * TG_KC + 16 * (4 * lg + t));
          const v4i aop = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
          acc[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop, acc[m], 0, 0, 0);
        }
      }
    }
  }
  // epilogue: lane holds rows `row`, tokens tok0 + 16m + 4*lg + r
  const bool rlive = row < a.out;
#pragma unroll
  for (int m = 0; m < MB; m++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t tk = tok0 + 16 * m + 4 * lg + r;
      const bool live = rlive && tk < a.seq;
      const uint32_t tkc = tk < a.seq ? tk : a.seq - 1;
      const float gm = a.gamma[tkc];
      // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
      const float val = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, gm), (float)(acc[m][r] >> 6)));
      if (EPI == NLG_EPI_STORE || EPI == NLG_EPI_ARGMAX) {
        if (live) a.y[(size_t)tk * a.ystride + row] = val;
      } else if (EPI == NLG_EPI_RESID) {
        if (live) a.y[(size_t)tk * a.ystride + row] = __fadd_rn(a.res[(size_t)tk * a.rstride + row], val);
      } else if (EPI == NLG_EPI_SWIGLU || EPI == NLG_EPI_QKV) {
        const float pv = __int_as_float(nlg_dpp<0xB1>(__float_as_int(val)));  // row ^ 1
        if (EPI == NLG_EPI_SWIGLU) {
          if (live && !(lane & 1)) {
            const float sg = 1.0f / (1.0f + expf(0.0f - val));
            a.y[(size_t)tk * a.ystride + (row >> 1)] = (val * sg) * pv;
          }
        } else if (live) {
          const int32_t pr = a.pos[0] + (a.qper ? (int32_t)(tk % a.qper) : 0);
          const bool pos_ok = pr >= 0 && (uint32_t)pr < a.max_seq;
          const uint32_t p = pos_ok ? (uint32_t)pr : 0u;
          const uint32_t sec = row < a.nq ? row : (row < a.nq + a.nkv ? row - a.nq : row - a.nq - a.nkv);
          const uint32_t dd = sec % a.hd, half = a.hd >> 1, ci = p * half + (dd >> 1);
          const float cs = a.co[ci], sn = a.si[ci];
          const bool odd = lane & 1;
          const float a0 = odd ? pv : val, a1 = odd ? val : pv;
          const float rot = odd ? __fadd_rn(__fmul_rn(a0, sn), __fmul_rn(a1, cs))
                                : __fsub_rn(__fmul_rn(a0, cs), __fmul_rn(a1, sn));
          if (row < a.nq) {
            a.y[(size_t)tk * a.ystride + row] = rot;
          } else if (pos_ok) {
            const bool isk = row < a.nq + a.nkv;
            const uint32_t kh = sec / a.hd, sq = a.qper ? tk / a.qper : tk;
            const size_t at = (((size_t)sq * a.kvheads + kh) * a.max_seq + p) * a.hd + dd;
            if (isk) a.kc[at] = __builtin_bit_cast(uint16_t, (_Float16)rot);
            else a.vc[at] = __builtin_bit_cast(uint16_t, (_Float16)val);
          }
        }
      }
      if (EPI == NLG_EPI_ARGMAX) {
        // first maximum over the wave's 16 rows for this token
        float bv = live && val == val ? val : -INFINITY;
        int32_t bi = live && val == val ? (int32_t)row : -1;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const float ov = __shfl_xor(bv, off);
          const int32_t oi = __shfl_xor(bi, off);
          if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
        }
        if (lr == 0) {
          s_bv[w][16 * m + 4 * lg + r] = bv;
          s_bi[w][16 * m + 4 * lg + r] = bi;
        }
      }
    }
  }
  if (EPI == NLG_EPI_ARGMAX) {
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < MT; t += 256) {
      float bv = s_bv[0][t];
      int32_t bi = s_bi[0][t];
      for (int k = 1; k < 4; k++) {
        const float ov = s_bv[k][t];
        const int32_t oi = s_bi[k][t];
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
      }
      const uint32_t tk = tok0 + t;
      if (tk < a.seq) {
        a.pval[(size_t)tk * a.nparts + blockIdx.x] = bv;
        a.pidx[(size_t)tk * a.nparts + blockIdx.x] = bi;
      }
    }
  }
}

// ------------------------------------------------------------ launchers

int nlg_act_q_launch(const float *x, const float *gain, float eps, const float *attn_mz, uint32_t attn_nc,
                     uint32_t hd, int pro, uint8_t *xq, float *gamma, uint32_t seq, uint32_t cols,
                     hipStream_t st) {
  if (!seq) return NLG_OK;
  if (cols % 64 || !cols || cols > 16384) return nlg_fail("act quant: cols must be a multiple of 64 in [64, 16384]");
  ActQArgs a{x, gain, eps, attn_mz, attn_nc, hd, xq, gamma, seq, cols};
  const dim3 grid(seq), blk(256);
#define AQ(P)                                                                                      \
  do {                                                                                             \
    if (cols <= 4096) hipLaunchKernelGGL((k_act_q<1, P>), grid, blk, 0, st, a);                    \
    else if (cols <= 8192) hipLaunchKernelGGL((k_act_q<2, P>), grid, blk, 0, st, a);               \
    else hipLaunchKernelGGL((k_act_q<4, P>), grid, blk, 0, st, a);                                 \
  } while (0)
  if (pro == NLG_PRO_RMS) AQ(NLG_PRO_RMS);
  else if (pro == NLG_PRO_ATTN) AQ(NLG_PRO_ATTN);
  else AQ(NLG_PRO_NONE);
#undef AQ
  NLG_LAUNCHED("activation quantisation");
  return NLG_OK;
}

int nlg_tgemm_launch(const GemmArgs &a0, int epi, hipStream_t st) {
  GemmArgs a = a0;
  if (!a.seq || !a.out) return NLG_OK;
  if (a.cols % TG_KC || !a.cols) return nlg_fail("ternary GEMM: cols must be a multiple of %d", TG_KC);
  if (((uintptr_t)a.w2 & 15) || ((uintptr_t)a.xq & 15)) return nlg_fail("ternary GEMM: 16-byte alignment");
  a.wng = a.cols / 16;
  // up to 32 tokens per workgroup: the 32 x 2064-byte activation block
  // stays under the 64 KiB a workgroup may hold
  const int MB = a.seq <= 16 ? 1 : 2;
  const uint32_t MT = 16u * MB;
  const dim3 grid(nlg_blocks(a.out, 64), (a.seq + MT - 1) / MT), blk(256);
  if (grid.y > 65535) return nlg_fail("ternary GEMM: seq too large");
  const size_t lds = (size_t)MT * TG_PITCH;
  if (epi == NLG_EPI_ARGMAX) a.nparts = grid.x;
  const int nph = a.cols <= 2048 ? 1 : (a.cols <= 4096 ? 2 : (a.cols <= 8192 ? 4 : 8));
#define TGP(M, E)                                                                                 \
  do {                                                                                            \
    if (nph == 1) hipLaunchKernelGGL((k_tgemm<M, 1, E>), grid, blk, lds, st, a);                  \
    else if (nph == 2) hipLaunchKernelGGL((k_tgemm<M, 2, E>), grid, blk, lds, st, a);             \
    else if (nph == 4) hipLaunchKernelGGL((k_tgemm<M, 4, E>), grid, blk, lds, st, a);             \
    else hipLaunchKernelGGL((k_tgemm<M, 8, E>), grid, blk, lds, st, a);                           \
  } while (0)
#define TG(E)                                                                                     \
  do {                                                                                            \
    if (MB == 1) TGP(1, E);                                                                       \
    else TGP(2, E);                                                                               \
  } while (0)
  switch (epi) {
    case NLG_EPI_STORE: TG(NLG_EPI_STORE); break;
    case NLG_EPI_RESID: TG(NLG_EPI_RESID); break;
    case NLG_EPI_SWIGLU: TG(NLG_EPI_SWIGLU); break;
    case NLG_EPI_QKV: TG(NLG_EPI_QKV); break;
    case NLG_EPI_ARGMAX: TG(NLG_EPI_ARGMAX); break;
    default: return nlg_fail("ternary GEMM: unknown epilogue %d", epi);
  }
#undef TG
#undef TGP
  NLG_LAUNCHED("ternary GEMM (int8 MFMA)");
  return NLG_OK;
}

bool nlg_batched(uint32_t seq, uint32_t cols) { return seq >= NLG_BATCHED_MIN && cols % TG_KC == 0; }

size_t nlg_batched_scratch_bytes(uint32_t seq, uint32_t cols) {
  return ((size_t)seq * cols + 255) / 256 * 256 + (size_t)seq * 4;
}

int nlg_batched_launch(const FusedArgs &f, int pro, int epi, hipStream_t st) {
  if (f.cols > 16384 || !f.cols) return nlg_fail("batched ternary linear: cols %u > 16384", f.cols);
  if (((uintptr_t)f.x & 15) || ((uintptr_t)f.w2 & 15) || (pro == NLG_PRO_RMS && ((uintptr_t)f.gain & 15)))
    return nlg_fail("batched ternary linear: x, w2 and gain must be 16-byte aligned");
  if ((epi == NLG_EPI_SWIGLU || epi == NLG_EPI_QKV) && f.out % 2)
    return nlg_fail("batched ternary linear: paired epilogues need an even row count");
  if (pro == NLG_PRO_ATTN &&
      (!f.hd || f.hd % 4 || f.cols % f.hd || !f.attn_nc || f.attn_nc > NLG_ATTN_MAX_CHUNKS || !f.attn_mz))
    return nlg_fail("batched ternary linear: bad attention partials");
  const size_t xq_bytes = ((size_t)f.seq * f.cols + 255) / 256 * 256;
  uint8_t *xq;
  if (f.act_scratch) {
    if (f.act_scratch_bytes < nlg_batched_scratch_bytes(f.seq, f.cols))
      return nlg_fail("batched ternary linear: scratch of %zu bytes is short", f.act_scratch_bytes);
    xq = (uint8_t *)f.act_scratch;
  } else {
    xq = (uint8_t *)nlg_scratch(nlg_batched_scratch_bytes(f.seq, f.cols), st);
    if (!xq) return NLG_ERR;
  }
  float *gamma = (float *)(xq + xq_bytes);
  if (nlg_act_q_launch(f.x, f.gain, f.eps, f.attn_mz, f.attn_nc, f.hd, pro, xq, gamma, f.seq, f.cols, st))
    return NLG_ERR;
  if (f.gamma_out) NLG_HIP(hipMemcpyAsync(f.gamma_out, gamma, (size_t)f.seq * 4, hipMemcpyDeviceToDevice, st));
  GemmArgs g{};
  g.xq = xq; g.gamma = gamma; g.w2 = f.w2; g.bias = f.bias; g.beta = f.beta; g.beta_per_row = f.beta_per_row;
  g.seq = f.seq; g.out = f.out; g.cols = f.cols; g.y = f.y; g.ystride = f.ystride; g.res = f.res;
  g.rstride = f.rstride; g.nq = f.nq; g.nkv = f.nkv; g.hd = f.hd; g.kvheads = f.kvheads; g.max_seq = f.max_seq;
  g.co = f.co; g.si = f.si; g.pos = f.pos; g.kc = f.kc; g.vc = f.vc; g.qper = f.qper;
  g.pval = f.pval; g.pidx = f.pidx;
  return nlg_tgemm_launch(g, epi, st);
}
