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
//
// 128 tokens and more (and 65+ tokens of many rows): k_tgemm_w (32 x 32 x
// 32 MFMAs; 256-row workgroups whose waves own 64 rows x 64 or 32 tokens,
// fed by direct global-to-LDS activation loads), for a few tiles of long
// rows with their columns split over gridDim.z slices.
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
  uint32_t stream_x;    // non-temporal loads of x (large row blocks)
};

// 256 threads per token row; thread t holds the row's float4s t + 256 j
// (j < 4 G16, cols <= 4096 G16), so every load of a wave reads 1 KiB
// contiguous.  A 16-column group's four float4s sit in the four lanes of a
// quad; each lane quantises its own word and the 4x4 byte transpose into
// matrix-core order runs across the quad (DPP broadcasts), each lane then
// storing one word of the group (256 contiguous bytes per wave store).
template <int G16, int PRO>
__global__ __launch_bounds__(256) void k_act_q(ActQArgs a) {
  constexpr int J = 4 * G16;
  __shared__ float red[4], red2[4];  // the two reductions' own scratch: no reuse barrier
  asm volatile("" ::"s"(a.x), "s"(a.gain), "s"(a.xq), "s"(a.gamma), "s"(a.cols));
  const uint32_t tok = blockIdx.x;
  const uint32_t nf4 = a.cols >> 2;
  float4 v[J];
  // PRO_ATTN3: exactly three chunks (see k_tern_fused's prologue)
  constexpr bool ATT = PRO == NLG_PRO_ATTN || PRO == NLG_PRO_ATTN3;
  constexpr int NC = PRO == NLG_PRO_ATTN3 ? 3 : NLG_ATTN_MAX_CHUNKS;
  if (ATT) {
    // attention merged from its chunks, in k_attn_merge's operation order
    const uint32_t heads = a.cols / a.hd;
    const float4 *c4 = (const float4 *)a.x;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const uint32_t f0 = threadIdx.x + 256u * j, f = f0 < nf4 ? f0 : nf4 - 1, h = (4 * f) / a.hd;
      float4 cx[NC];
      float2 mz[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const uint32_t cc = (uint32_t)c < a.attn_nc ? (uint32_t)c : a.attn_nc - 1;
        const size_t tc = (size_t)tok * a.attn_nc + cc;
        cx[c] = c4[tc * nf4 + f];
        mz[c] = *(const float2 *)(a.attn_mz + (tc * heads + h) * 2);
      }
      float mm = -1.0e30f;
#pragma unroll
      for (int c = 0; c < NC; c++) mm = mz[c].x > mm ? mz[c].x : mm;
      float zz = 0.0f;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const float sc = (uint32_t)c < a.attn_nc ? nlg_exp2(mz[c].x - mm) : 0.0f;  // base-2 maxima
        zz = fmaf(mz[c].y, sc, zz);
        acc.x = fmaf(cx[c].x, sc, acc.x);
        acc.y = fmaf(cx[c].y, sc, acc.y);
        acc.z = fmaf(cx[c].z, sc, acc.z);
        acc.w = fmaf(cx[c].w, sc, acc.w);
      }
      v[j] = make_float4(acc.x / zz, acc.y / zz, acc.z / zz, acc.w / zz);
    }
  } else {
    // A large row block is read once and streams from HBM: non-temporal
    // loads (16,384 x 6,912: 105 -> 91 us, the GEMM after it unchanged).  A
    // small one was just written by the previous launch and sits in the
    // caches, where non-temporal loads were slower (batch-32 decode: the
    // down projection's pair 9.93 -> 10.46 us).
    const float4 *x4 = (const float4 *)(a.x + (size_t)tok * a.cols);
    if (a.stream_x) {
#pragma unroll
      for (int j = 0; j < J; j++) {
        const uint32_t f0 = threadIdx.x + 256u * j;
        v[j] = nlg_ld_stream_f4(&x4[f0 < nf4 ? f0 : nf4 - 1]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < J; j++) {
        const uint32_t f0 = threadIdx.x + 256u * j;
        v[j] = x4[f0 < nf4 ? f0 : nf4 - 1];
      }
    }
  }
  float4 gv[J];
  if (PRO == NLG_PRO_RMS) {
    const float4 *g4 = (const float4 *)a.gain;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const uint32_t f0 = threadIdx.x + 256u * j;
      gv[j] = g4[f0 < nf4 ? f0 : nf4 - 1];
    }
  }
#pragma unroll
  for (int j = 0; j < J; j++)
    if (threadIdx.x + 256u * j >= nf4) v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (PRO == NLG_PRO_RMS) {
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
      sq = sq + v[j].x * v[j].x;
      sq = sq + v[j].y * v[j].y;
      sq = sq + v[j].z * v[j].z;
      sq = sq + v[j].w * v[j].w;
    }
    sq = nlg_block_sum_f32<4, true>(sq, red);
    sq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq)));
    const float istd = 1.0f / sqrtf(sq / (float)a.cols + a.eps);
#pragma unroll
    for (int j = 0; j < J; j++) {
      v[j].x = (v[j].x * istd) * gv[j].x;
      v[j].y = (v[j].y * istd) * gv[j].y;
      v[j].z = (v[j].z * istd) * gv[j].z;
      v[j].w = (v[j].w * istd) * gv[j].w;
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < J; j++) {
    float t;
    t = dsl_abs(v[j].x); amax = t > amax ? t : amax;
    t = dsl_abs(v[j].y); amax = t > amax ? t : amax;
    t = dsl_abs(v[j].z); amax = t > amax ? t : amax;
    t = dsl_abs(v[j].w); amax = t > amax ? t : amax;
  }
  amax = nlg_block_max_f32<4, true>(amax, red2);
  const float g = nlg_gamma_of(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(amax))));
  const float ginv = 1.0f / g;
  const bool fast = quant_fast(g);
  if (threadIdx.x == 0) a.gamma[tok] = g;
  // Lane i of a quad holds the group's word n_i (its columns 4i..4i+3) and
  // writes y_i = (n0.b_i, n1.b_i, n2.b_i, n3.b_i): byte i of each word.
  const uint32_t i = threadIdx.x & 3u;
  const uint32_t sel_lo = 0x0c0c0000u | ((4u + i) << 8) | i, sel_hi = 0x00000c0cu | ((4u + i) << 24) | (i << 16);
  uint32_t *dst = (uint32_t *)(a.xq + (size_t)tok * a.cols);
  uint32_t qw[J];
  quant_words<J>(v, g, ginv, fast, qw);
#pragma unroll
  for (int j = 0; j < J; j++) {
    const uint32_t f = threadIdx.x + 256u * j;
    const uint32_t n0 = nlg_qperm<0x00>(qw[j]), n1 = nlg_qperm<0x55>(qw[j]);
    const uint32_t n2 = nlg_qperm<0xAA>(qw[j]), n3 = nlg_qperm<0xFF>(qw[j]);
    const uint32_t y = __builtin_amdgcn_perm(n1, n0, sel_lo) | __builtin_amdgcn_perm(n3, n2, sel_hi);
    if (f < nf4) dst[f] = y;
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
  // k_tgemm_w split over the columns: gridDim.z slices of the chunks, each
  // slice's int32 accumulators to ksum (one block of registers per
  // (slice, tile, thread)), tile arrivals counted in kctr (zero between
  // launches); the last slice of a tile to arrive adds the others' and
  // runs the epilogue
  int32_t *ksum;
  uint32_t *kctr;
  bool allow_split;  // the launcher may take split workspace from the library
};

// One output element of the batched linear (every lane calls it: the SwiGLU
// and RoPE pairs are exchanged across lanes l, l^1, which hold rows 2j, 2j+1).
// Best (value, index) over the 16 lanes of each DPP row -- the larger value,
// the lower index among equals; index -1: no candidate -- in every lane of
// the row.  That order is total, so any pairing finds the same winner: the
// quad swaps, then the half-row and row mirrors (each pairs every lane with
// one of the other quad, then of the other half).  DPP moves, not LDS
// permutes: each step is a few VALU cycles instead of an LDS round trip.
__device__ __forceinline__ void row16_argmax(float &bv, int32_t &bi) {
#define R16_STEP(C)                                                                          \
  {                                                                                          \
    const float ov = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(bv), C, 0xf, 0xf, true)); \
    const int32_t oi = __builtin_amdgcn_mov_dpp(bi, C, 0xf, 0xf, true);                     \
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {                          \
      bv = ov;                                                                               \
      bi = oi;                                                                               \
    }                                                                                        \
  }
  R16_STEP(0xB1)   // quad_perm [1,0,3,2]
  R16_STEP(0x4E)   // quad_perm [2,3,0,1]
  R16_STEP(0x141)  // row_half_mirror
  R16_STEP(0x140)  // row_mirror
#undef R16_STEP
}

// the epilogue operands of one (token, row), fetched before the main loop
struct TgPre {
  float res, cs, sn;
  uint32_t p;
  bool pos_ok;
};

template <int EPI>
__device__ __forceinline__ TgPre tg_prefetch(const GemmArgs &a, uint32_t rowc, uint32_t tk) {
  TgPre r{0.0f, 0.0f, 0.0f, 0u, false};
  const uint32_t tkc = tk < a.seq ? tk : a.seq - 1;
  if (EPI == NLG_EPI_RESID) r.res = a.res[(size_t)tkc * a.rstride + rowc];
  if (EPI == NLG_EPI_QKV) {
    const int32_t pr = nlg_ld_uniform_i32(a.pos) + (a.qper ? (int32_t)(tkc % a.qper) : 0);
    r.pos_ok = pr >= 0 && (uint32_t)pr < a.max_seq;
    r.p = r.pos_ok ? (uint32_t)pr : 0u;
    const uint32_t sec = rowc < a.nq ? rowc : (rowc < a.nq + a.nkv ? rowc - a.nq : rowc - a.nq - a.nkv);
    const uint32_t ci = r.p * (a.hd >> 1) + ((sec % a.hd) >> 1);
    r.cs = a.co[ci];
    r.sn = a.si[ci];
  }
  return r;
}

template <int EPI>
__device__ __forceinline__ void tg_store_pre(const GemmArgs &a, int lane, uint32_t row, uint32_t tk, bool live,
                                             float val, const TgPre &pre) {
  if (EPI == NLG_EPI_STORE || EPI == NLG_EPI_ARGMAX) {
    if (live) a.y[(size_t)tk * a.ystride + row] = val;
  } else if (EPI == NLG_EPI_RESID) {
    if (live) a.y[(size_t)tk * a.ystride + row] = __fadd_rn(pre.res, val);
  } else if (EPI == NLG_EPI_SWIGLU || EPI == NLG_EPI_QKV) {
    const float pv = __int_as_float(nlg_dpp<0xB1>(__float_as_int(val)));  // row ^ 1
    if (EPI == NLG_EPI_SWIGLU) {
      if (live && !(lane & 1)) {
        const float sg = nlg_silu_gate(val);
        a.y[(size_t)tk * a.ystride + (row >> 1)] = (val * sg) * pv;
      }
    } else if (live) {
      const uint32_t sec = row < a.nq ? row : (row < a.nq + a.nkv ? row - a.nq : row - a.nq - a.nkv);
      const uint32_t dd = sec % a.hd;
      const bool odd = lane & 1;
      const float a0 = odd ? pv : val, a1 = odd ? val : pv;
      const float rot = odd ? __fadd_rn(__fmul_rn(a0, pre.sn), __fmul_rn(a1, pre.cs))
                            : __fsub_rn(__fmul_rn(a0, pre.cs), __fmul_rn(a1, pre.sn));
      if (row < a.nq) {
        a.y[(size_t)tk * a.ystride + row] = rot;
      } else if (pre.pos_ok) {
        const bool isk = row < a.nq + a.nkv;
        const uint32_t kh = sec / a.hd, sq = a.qper ? tk / a.qper : tk;
        const size_t at = (((size_t)sq * a.kvheads + kh) * a.max_seq + pre.p) * a.hd + dd;
        if (isk) a.kc[at] = __builtin_bit_cast(uint16_t, (_Float16)rot);
        else a.vc[at] = __builtin_bit_cast(uint16_t, (_Float16)val);
      }
    }
  }
}

// the same with the operands fetched here (row < out, tk < seq where live)
template <int EPI>
__device__ __forceinline__ void tg_store(const GemmArgs &a, int lane, uint32_t row, uint32_t tk, bool live,
                                         float val) {
  tg_store_pre<EPI>(a, lane, row, tk, live, val, tg_prefetch<EPI>(a, row < a.out ? row : a.out - 1, tk));
}

#define TG_KC 256                 // columns per chunk (16 2-bit words of a row)
#define TG_PH 8                   // chunks per phase
#define TG_PITCH (TG_PH * TG_KC + 16)  // LDS row pitch in bytes (staggers the banks)

// MB: 16-token blocks per workgroup (MT = 16*MB tokens).  The columns go in
// phases of 8 chunks (2048 columns): at the start of a phase every lane issues
// the loads of its weight row's 8 chunks (registers) and the workgroup's
// MT x 2048 activation block (to LDS), so a phase costs one memory round
// trip; then 8 x 4 x MB matrix-core steps run out of registers and LDS.
// NPH: phases (compile-time, so the loop over them unrolls and the staging
// arrays stay in registers) of PH chunks: cols <= 256 * PH * NPH.  The
// epilogue's operands (gamma, the residual, RoPE entries) are fetched
// before the first phase, not after the last.
// With TILED, a.w2 is the registered tiled copy (laid out for k_tgemm_w's
// loads): lane (lg, lr)'s
// 16 bytes of chunk c (words 4 lg .. 4 lg + 3 of its row, the row layout's
// wrow[4 c + lg]) are unit 128 c + 64 (lg % 2) + 32 (lg / 2) + row % 32 of its
// 32-row block's tiles, so a load instruction reads four 256-byte runs.
__device__ __forceinline__ const uint4 *tg_wbase(const GemmArgs &a, uint32_t rowc, int lg, bool tiled) {
  if (tiled)
    return (const uint4 *)a.w2 + (size_t)(rowc / 32) * (a.cols / TG_KC) * 128 + 64 * (lg & 1) + 32 * (lg >> 1) +
           rowc % 32;
  return (const uint4 *)(a.w2 + (size_t)rowc * a.wng) + lg;
}

template <int MB, int NPH, int PH, int EPI, bool TILED = false>
__global__ __launch_bounds__(256) void k_tgemm(GemmArgs a) {
  constexpr int MT = 16 * MB;
  constexpr int PITCH = PH * TG_KC + 16;  // LDS row pitch in bytes (staggers the banks)
  extern __shared__ __align__(16) uint8_t s_a[];  // MT x PITCH
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
  const uint4 *wrow = tg_wbase(a, rowc, lg, TILED);
  constexpr uint32_t WCS = TILED ? 128 : 4;  // uint4s from one chunk to the next
  // activation staging: piece p = threadIdx.x + 256 i is token p / SL,
  // 16-byte slot p % SL of the phase's 256 PH columns
  constexpr int SL = PH * TG_KC / 16;          // slots per token row
  constexpr int NA = MT * SL / 256;            // pieces per thread
  static_assert(MT * SL % 256 == 0, "whole staging pieces per thread");
  const float bo_raw = (a.bias ? a.bias : a.beta)[a.bias ? rowc : 0];
  const float be = a.beta[a.beta_per_row ? rowc : 0];
  const float bo = a.bias ? bo_raw : 0.0f;
  // epilogue operands of the lane's (token, row) pairs
  float gm[MB][4];
  TgPre pre[MB][4];
#pragma unroll
  for (int m = 0; m < MB; m++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t tk = tok0 + 16 * m + 4 * lg + r;
      gm[m][r] = a.gamma[tk < a.seq ? tk : a.seq - 1];
      pre[m][r] = tg_prefetch<EPI>(a, rowc, tk);
    }
  v4i acc[MB];
#pragma unroll
  for (int m = 0; m < MB; m++) acc[m] = (v4i){0, 0, 0, 0};
  // The staging registers are ext_vector values indexed by constants, not
  // arrays: an array here ends up in scratch once the phase loop unrolls.
  typedef uint32_t wvec_t __attribute__((ext_vector_type(4 * PH)));
  typedef uint32_t avec_t __attribute__((ext_vector_type(4 * NA)));
#pragma unroll
  for (int ph = 0; ph < NPH; ph++) {
    const uint32_t c0 = ph * PH;
    if (c0 >= nchunks) break;  // uniform
    wvec_t wv;
#pragma unroll
    for (int i = 0; i < PH; i++) {
      const uint32_t cc = c0 + i < nchunks ? c0 + i : nchunks - 1;
      const uint4 u = wrow[WCS * cc];
      // chunks past the end contribute zero
      const uint32_t keep = c0 + i < nchunks ? 0xffffffffu : 0u;
      wv[4 * i + 0] = u.x & keep;
      wv[4 * i + 1] = u.y & keep;
      wv[4 * i + 2] = u.z & keep;
      wv[4 * i + 3] = u.w & keep;
    }
    avec_t ar;
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const uint32_t p = threadIdx.x + 256u * i, t = p / SL, slot = p % SL;
      const uint32_t tk = tok0 + t < a.seq ? tok0 + t : a.seq - 1;
      const uint32_t col = c0 * TG_KC + 16 * slot;
      const uint32_t colc = col < a.cols ? col : a.cols - 16;
      const uint4 u = *(const uint4 *)(a.xq + (size_t)tk * a.cols + colc);
      ar[4 * i + 0] = u.x;
      ar[4 * i + 1] = u.y;
      ar[4 * i + 2] = u.z;
      ar[4 * i + 3] = u.w;
    }
    if (c0) __syncthreads();  // every wave is done with the previous phase's block
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const uint32_t p = threadIdx.x + 256u * i;
      *(uint4 *)(&s_a[(p / SL) * PITCH + 16 * (p % SL)]) = make_uint4(ar[4 * i], ar[4 * i + 1], ar[4 * i + 2], ar[4 * i + 3]);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PH; i++) {
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t wd = wv[4 * i + t];
        const v4i bop = {(int)((wd << 6) & 0xC0C0C0C0u), (int)((wd << 4) & 0xC0C0C0C0u),
                         (int)((wd << 2) & 0xC0C0C0C0u), (int)(wd & 0xC0C0C0C0u)};
#pragma unroll
        for (int m = 0; m < MB; m++) {
          const uint4 av = *(const uint4 *)(s_a + (16 * m + lr) * PITCH + i * TG_KC + 16 * (4 * lg + t));
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
      // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
      const float val = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, gm[m][r]), (float)(acc[m][r] >> 6)));
      tg_store_pre<EPI>(a, lane, row, tk, live, val, pre[m][r]);
      if (EPI == NLG_EPI_ARGMAX) {
        // first maximum over the wave's 16 rows for this token
        float bv = live && val == val ? val : -INFINITY;
        int32_t bi = live && val == val ? (int32_t)row : -1;
        row16_argmax(bv, bi);
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

// ------------------------------------------------------------ k_tgemm_k
//
// Few tokens (decode batches): the 64-row workgroups of k_tgemm leave most
// CUs idle, so here a workgroup owns 16 output rows x 16 MB tokens and its
// four waves split the columns: wave w takes chunks w*per .. (w+1)*per - 1
// (per = ceil(chunks / 4) <= PM) and loads its operands straight from global
// memory into registers in matrix-core order (no LDS stage, no barrier
// until the end).  A wave's weights are short (one 16-byte load per chunk),
// so all PM of them are issued first, then the epilogue's operands (gamma,
// bias, beta, the residual, the RoPE table entries): the kernel pays one HBM
// round trip.  The activations (shared by every workgroup, so L2-resident)
// run TK_D chunks ahead of the matrix cores.  Steps past the wave's range
// load a valid chunk and mask its weights to zero.  The four int32 partial
// sums meet in LDS (integer adds: exact in any order) and wave w finishes
// accumulator register w of every token block.

#define TK_D 3  // activation chunks in flight
#define TK_PITCH 68  // LDS row pitch (words) of a wave's activation tile: 256 bytes + 16

template <int MB, int EPI, int PM, bool TILED = false>
__global__ __launch_bounds__(256) void k_tgemm_k(GemmArgs a) {
  constexpr int NA = 4 * MB;  // 16-byte activation pieces per lane and chunk
  constexpr int D = PM < TK_D ? PM : TK_D;
  typedef uint32_t avec __attribute__((ext_vector_type(4 * NA)));
  __shared__ v4i s_red[4][MB][64];
  // each wave's activation tile of one chunk: MB blocks x 16 tokens x 256
  // bytes, rows padded to TK_PITCH words
  __shared__ __align__(16) uint32_t s_at[4][MB][16][TK_PITCH];
  asm volatile("" ::"s"(a.xq), "s"(a.gamma), "s"(a.w2), "s"(a.bias), "s"(a.beta), "s"(a.y), "s"(a.seq),
               "s"(a.out), "s"(a.cols), "s"(a.wng), "s"(a.ystride), "s"(a.beta_per_row));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t row = blockIdx.x * 16 + lr;  // this lane's output row (B column j)
  const uint32_t rowc = row < a.out ? row : a.out - 1;
  const uint32_t tok0 = blockIdx.y * 16 * MB;
  const uint32_t nchunks = a.cols / TG_KC;
  const uint32_t per = (nchunks + 3) / 4, cb = w * per;
  const uint32_t ce = min(cb + per, nchunks);
  const uint4 *wrow = tg_wbase(a, rowc, lg, TILED);
  constexpr uint32_t WCS = TILED ? 128 : 4;  // uint4s from one chunk to the next
  // Activations are fetched whole rows at a time -- load u of block m brings
  // token 16 m + 4 u + lane / 16, bytes 16 (lane % 16) of a chunk, so each
  // instruction reads four full 256-byte row chunks -- and reach the matrix
  // cores' layout (lane (i, g) at step t: token i, bytes 64 g + 16 t) through
  // the wave's LDS tile.  Fetched in that layout directly, one instruction
  // touched 16 rows in 16-byte pieces: twice the cache lines, each half used,
  // for data every workgroup re-reads.
  const uint8_t *xa[MB][4];
#pragma unroll
  for (int m = 0; m < MB; m++)
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t tk = tok0 + 16 * m + 4 * u + (lane >> 4);
      xa[m][u] = a.xq + (size_t)(tk < a.seq ? tk : a.seq - 1) * a.cols + 16 * (lane & 15);
    }
  // 1. the lane's 4 weight words (64 columns of its row) of every chunk
  uint4 wq[PM];
#pragma unroll
  for (int j = 0; j < PM; j++) {
    const uint32_t c = cb + j;
    wq[j] = nlg_ld_stream(&wrow[WCS * (c < ce ? c : nchunks - 1)]);
  }
  // 2. the first D chunks' activations, whole rows per load (see above)
  avec av[PM];
#define TK_LOADA(k)                                                                       \
  do {                                                                                    \
    const uint32_t c = cb + (k);                                                          \
    const uint32_t cc = c < ce ? c : nchunks - 1;                                         \
    _Pragma("unroll") for (int m = 0; m < MB; m++) {                                      \
      _Pragma("unroll") for (int u = 0; u < 4; u++) {                                     \
        const uint4 v = *(const uint4 *)(xa[m][u] + (size_t)cc * TG_KC);                   \
        av[k][16 * m + 4 * u] = v.x; av[k][16 * m + 4 * u + 1] = v.y;                     \
        av[k][16 * m + 4 * u + 2] = v.z; av[k][16 * m + 4 * u + 3] = v.w;                 \
      }                                                                                   \
    }                                                                                     \
  } while (0)
#pragma unroll
  for (int k = 0; k < D; k++) TK_LOADA(k);
  // 3. the epilogue's operands: wave w finishes token tok0 + 16 m + 4 lg + w
  const float bo_raw = (a.bias ? a.bias : a.beta)[a.bias ? rowc : 0];
  const float be = a.beta[a.beta_per_row ? rowc : 0];
  float gm[MB];
  TgPre pre[MB];
#pragma unroll
  for (int m = 0; m < MB; m++) {
    const uint32_t tk = tok0 + 16 * m + 4 * lg + w;
    gm[m] = a.gamma[tk < a.seq ? tk : a.seq - 1];
    pre[m] = tg_prefetch<EPI>(a, rowc, tk);
  }
  // keep every load above issued here: the scheduler would otherwise sink
  // weight loads into the loop (to save registers) and pay HBM latency there
  __builtin_amdgcn_sched_barrier(0);
  // 4. the matrix-core steps, activations D chunks ahead
  v4i acc[MB];
#pragma unroll
  for (int m = 0; m < MB; m++) acc[m] = (v4i){0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < PM; k++) {
    if (k + D < PM) TK_LOADA(k + D);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t keep = cb + k < ce ? 0xffffffffu : 0u;
    // chunk k through the wave's tile: rows in, matrix-core layout out (one
    // wave's LDS operations run in order, so no barrier is needed)
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
      for (int u = 0; u < 4; u++)
        *(uint4 *)&s_at[w][m][4 * u + (lane >> 4)][4 * (lane & 15)] =
            make_uint4(av[k][16 * m + 4 * u], av[k][16 * m + 4 * u + 1], av[k][16 * m + 4 * u + 2],
                       av[k][16 * m + 4 * u + 3]);
    uint4 at[MB][4];
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
      for (int t = 0; t < 4; t++) at[m][t] = *(const uint4 *)&s_at[w][m][lr][4 * (4 * lg + t)];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t wd = (t == 0 ? wq[k].x : t == 1 ? wq[k].y : t == 2 ? wq[k].z : wq[k].w) & keep;
      const v4i bop = {(int)((wd << 6) & 0xC0C0C0C0u), (int)((wd << 4) & 0xC0C0C0C0u),
                       (int)((wd << 2) & 0xC0C0C0C0u), (int)(wd & 0xC0C0C0C0u)};
#pragma unroll
      for (int m = 0; m < MB; m++) {
        const v4i aop = {(int)at[m][t].x, (int)at[m][t].y, (int)at[m][t].z, (int)at[m][t].w};
        acc[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop, acc[m], 0, 0, 0);
      }
    }
  }
#undef TK_LOADA
#pragma unroll
  for (int m = 0; m < MB; m++) s_red[w][m][lane] = acc[m];
  __syncthreads();
  // wave w: register r = w of each token block (token tok0 + 16 m + 4 lg + w)
  const bool rlive = row < a.out;
  const float bo = a.bias ? bo_raw : 0.0f;
#pragma unroll
  for (int m = 0; m < MB; m++) {
    const int32_t q = s_red[0][m][lane][w] + s_red[1][m][lane][w] + s_red[2][m][lane][w] + s_red[3][m][lane][w];
    const uint32_t tk = tok0 + 16 * m + 4 * lg + w;
    const bool live = rlive && tk < a.seq;
    // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
    const float val = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, gm[m]), (float)(q >> 6)));
    tg_store_pre<EPI>(a, lane, row, tk, live, val, pre[m]);
  }
}

// ------------------------------------------------------------ k_tgemm_w

typedef int v16i __attribute__((ext_vector_type(16)));

// Column slices of one tile meet here (k_tgemm_w's split form).  Every
// slice leaves its accumulators in its own block of ksum with
// agent-coherent (write-through) stores, waits for them to
// complete, and counts itself in; the last to arrive reads the other
// slices' blocks (agent-coherent loads, past any stale L2 copy), adds them
// -- integer sums, the same in any order -- and returns true to run the
// epilogue.  It also re-zeros the tile's counter for the next launch,
// which the stream orders after this one.  s_last: one LDS word.
template <int MB, int NB>
__device__ __forceinline__ bool tl_split_meet(const GemmArgs &a, v16i (&acc)[MB][NB], uint32_t *s_last) {
  constexpr int NR = MB * NB * 16;  // accumulators per thread
  const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x, ntile = gridDim.x * gridDim.y, ks = gridDim.z;
  const size_t nthr = blockDim.x;
  // register j of every thread side by side: each store and load of a
  // wave covers 256 contiguous bytes
  int32_t *mine = a.ksum + ((size_t)blockIdx.z * ntile + tile) * NR * nthr + threadIdx.x;
#pragma unroll
  for (int mt = 0; mt < MB; mt++)
#pragma unroll
    for (int nt = 0; nt < NB; nt++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        __hip_atomic_store(mine + ((mt * NB + nt) * 16 + r) * nthr, acc[mt][nt][r], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t n = __hip_atomic_fetch_add(a.kctr + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = n + 1 == ks;
    if (n + 1 == ks) __hip_atomic_store(a.kctr + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!*s_last) return false;
  for (uint32_t z = 0; z < ks; z++) {
    if (z == blockIdx.z) continue;
    const int32_t *other = a.ksum + ((size_t)z * ntile + tile) * NR * nthr + threadIdx.x;
#pragma unroll
    for (int mt = 0; mt < MB; mt++)
#pragma unroll
      for (int nt = 0; nt < NB; nt++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          acc[mt][nt][r] += __hip_atomic_load(other + ((mt * NB + nt) * 16 + r) * nthr, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
  }
  return true;
}

// The epilogue of k_tgemm_w: acc[mt][nt] of lane (li, lg) of the wave (MB
// token blocks from token tok0 + 64 wm; the kernel passes wm = 0), rows
// rw[nt] (clamped rc[nt]), with bias bo and beta be per row block and the
// workgroup's gammas in s_gm.
//
// QKV: s_tp holds each of the workgroup's 128 tokens' cache position (-1
// where it is past max_seq) and s_tb its cache row's element offset
// ((sequence x kvheads x max_seq + position) x head_dim), computed once per
// workgroup; a row block's section, head and dimension once per block.
template <int MB, int NB, int EPI>
__device__ __forceinline__ void tl_epilogue(const GemmArgs &a, const v16i (&acc)[MB][NB], const uint32_t (&rw)[NB],
                                            const uint32_t (&rc)[NB], const float (&bo)[NB], const float (&be)[NB],
                                            const float *s_gm, int lane, int wm, int lg, uint32_t tok0,
                                            const int32_t *s_tp, const uint64_t *s_tb) {
  // acc[mt][nt] register r is token tok0 + 64 wm + 32 mt + (r%4) + 8 (r/4) + 4 lg,
  // row rw[nt].  gamma comes from LDS; the residual and RoPE
  // operands of a (token block, row block) are all fetched before its first
  // result is stored.  (y may be the residual itself, so the compiler keeps
  // every load behind the stores before it: fetched beside its own store,
  // each operand cost a memory round trip.  Measured at 16,384 tokens: the
  // gate|up GEMM 813 -> 746 us, its STORE form 881 -> 712 us.)
  if (EPI == NLG_EPI_SWIGLU) {
    // Gate row 2j and up row 2j+1 sit in lanes l, l^1.  Each lane of a pair
    // finishes half of the pair's tokens: the even lane registers 0..7, the
    // odd lane 8..15, after swapping the other half's value with its partner.
    const bool odd = lane & 1;
#pragma unroll
    for (int mt = 0; mt < MB; mt++) {
#pragma unroll
      for (int nt = 0; nt < NB; nt++) {
        const v16i q = acc[mt][nt];
        const bool lr = rw[nt] < a.out;
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const uint32_t tlo = tok0 + 64 * wm + 32 * mt + (k % 4) + 8 * (k / 4) + 4 * lg;
          const uint32_t thi = tlo + 16;  // register k + 8
          const float glo = s_gm[tlo - tok0], ghi = s_gm[thi - tok0];
          // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
          const float vlo = __fadd_rn(bo[nt], __fmul_rn(__fmul_rn(be[nt], glo), (float)(q[k] >> 6)));
          const float vhi = __fadd_rn(bo[nt], __fmul_rn(__fmul_rn(be[nt], ghi), (float)(q[k + 8] >> 6)));
          const float keep = odd ? vhi : vlo, give = odd ? vlo : vhi;
          const float got = __int_as_float(nlg_dpp<0xB1>(__float_as_int(give)));  // from lane ^ 1
          const float g = odd ? got : keep, u = odd ? keep : got;
          const uint32_t tk = odd ? thi : tlo;
          if (lr && tk < a.seq) {
            const float sg = nlg_silu_gate(g);
            a.y[(size_t)tk * a.ystride + (rw[nt] >> 1)] = (g * sg) * u;
          }
        }
      }
    }
    return;
  }
  if (EPI == NLG_EPI_ARGMAX) {
    // The logits, and per token the wave's (max, first index) over its 64
    // rows -- rbase = rw[0] - li .. + 63, partial rbase / 64, where k_tgemm's
    // 64-row workgroup puts it -- for the sampler.  A lane's two row blocks,
    // then the 16 lanes of its DPP row, then the wave's two rows of each
    // token half (lanes 0 and 16: tokens of lg = 0; 32 and 48: lg = 1).
    const uint32_t t64 = (rw[0] - (uint32_t)(lane & 31)) / 64;
#pragma unroll
    for (int mt = 0; mt < MB; mt++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const uint32_t tk = tok0 + 64 * wm + 32 * mt + (r % 4) + 8 * (r / 4) + 4 * lg;
        float bv = -INFINITY;
        int32_t bi = -1;
#pragma unroll
        for (int nt = 0; nt < NB; nt++) {
          // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
          const float v =
              __fadd_rn(bo[nt], __fmul_rn(__fmul_rn(be[nt], s_gm[tk - tok0]), (float)(acc[mt][nt][r] >> 6)));
          const bool live = rw[nt] < a.out && tk < a.seq;
          if (live) a.y[(size_t)tk * a.ystride + rw[nt]] = v;
          if (live && v == v && (bi < 0 || v > bv)) {  // rows ascend with nt: ties keep the first
            bv = v;
            bi = (int32_t)rw[nt];
          }
        }
        row16_argmax(bv, bi);
        const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
        const float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 16));
        const float v2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 32));
        const float v3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 48));
        const int32_t i0 = __builtin_amdgcn_readlane(bi, 0), i1 = __builtin_amdgcn_readlane(bi, 16);
        const int32_t i2 = __builtin_amdgcn_readlane(bi, 32), i3 = __builtin_amdgcn_readlane(bi, 48);
        const bool t1 = i1 >= 0 && (i0 < 0 || v1 > v0 || (v1 == v0 && i1 < i0));
        const bool t3 = i3 >= 0 && (i2 < 0 || v3 > v2 || (v3 == v2 && i3 < i2));
        const float wv = lg ? (t3 ? v3 : v2) : (t1 ? v1 : v0);
        const int32_t wi = lg ? (t3 ? i3 : i2) : (t1 ? i1 : i0);
        if ((lane & 31) == 0 && tk < a.seq && t64 < a.nparts) {
          a.pval[(size_t)tk * a.nparts + t64] = wv;
          a.pidx[(size_t)tk * a.nparts + t64] = wi;
        }
      }
    }
    return;
  }
  if (EPI == NLG_EPI_QKV) {
    const uint32_t half = a.hd >> 1;
    const bool odd = lane & 1;
#pragma unroll
    for (int nt = 0; nt < NB; nt++) {
      const uint32_t row = rw[nt], rcn = rc[nt];
      const uint32_t sec = rcn < a.nq ? rcn : (rcn < a.nq + a.nkv ? rcn - a.nq : rcn - a.nq - a.nkv);
      const uint32_t dd = sec % a.hd, kh = sec / a.hd, cd = dd >> 1;
      const bool isq = row < a.nq, isk = row < a.nq + a.nkv;
      uint16_t *const cache = (isk ? a.kc : a.vc) + ((size_t)kh * a.max_seq * a.hd + dd);
#pragma unroll
      for (int mt = 0; mt < MB; mt++) {
        float cs[16], sn[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int32_t p = s_tp[64 * wm + 32 * mt + (r % 4) + 8 * (r / 4) + 4 * lg];
          const uint32_t ci = (p >= 0 ? (uint32_t)p : 0u) * half + cd;
          cs[r] = a.co[ci];
          sn[r] = a.si[ci];
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const uint32_t t = 64 * wm + 32 * mt + (r % 4) + 8 * (r / 4) + 4 * lg, tk = tok0 + t;
          // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
          const float val =
              __fadd_rn(bo[nt], __fmul_rn(__fmul_rn(be[nt], s_gm[t]), (float)(acc[mt][nt][r] >> 6)));
          // decode-rope on the (row, row ^ 1) pair: C[i0] = a0*cc - a1*ss; C[i1] = a0*ss + a1*cc
          const float pv = __int_as_float(nlg_dpp<0xB1>(__float_as_int(val)));
          const float a0 = odd ? pv : val, a1 = odd ? val : pv;
          const float rot = odd ? __fadd_rn(__fmul_rn(a0, sn[r]), __fmul_rn(a1, cs[r]))
                                : __fsub_rn(__fmul_rn(a0, cs[r]), __fmul_rn(a1, sn[r]));
          if (row < a.out && tk < a.seq) {
            const int32_t p = s_tp[t];
            if (isq) {
              a.y[(size_t)tk * a.ystride + row] = rot;
            } else if (p >= 0) {
              cache[s_tb[t]] = __builtin_bit_cast(uint16_t, (_Float16)(isk ? rot : val));
            }
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MB; mt++) {
#pragma unroll
    for (int nt = 0; nt < NB; nt++) {
      TgPre pre[16];
#pragma unroll
      for (int r = 0; r < 16; r++)
        pre[r] = tg_prefetch<EPI>(a, rc[nt], tok0 + 64 * wm + 32 * mt + (r % 4) + 8 * (r / 4) + 4 * lg);
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const uint32_t tk = tok0 + 64 * wm + 32 * mt + (r % 4) + 8 * (r / 4) + 4 * lg;
        // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
        const float v =
            __fadd_rn(bo[nt], __fmul_rn(__fmul_rn(be[nt], s_gm[tk - tok0]), (float)(acc[mt][nt][r] >> 6)));
        tg_store_pre<EPI>(a, lane, rw[nt], tk, rw[nt] < a.out && tk < a.seq, v, pre[r]);
      }
    }
  }
}

// Many tokens, wide waves: a workgroup owns 256 output rows x MT = 32 MB
// tokens (the launcher runs MB = 2, or 1 for smaller grids), each of its 4
// waves 64 rows (two 32-row blocks) x all MT tokens (MB 32-token blocks).
// Every weight chunk is fetched once per workgroup (each wave owns its own
// rows) and every decoded B operand feeds MB MFMAs.  Activations go from global memory
// straight to LDS (global_load_lds_dwordx4: no staging registers, no LDS
// stores) into two [MT tokens][256 B] stages, one chunk ahead; their
// 16-byte units are XOR-swizzled by token (unit u of token k at slot
// u ^ (k % 16)), so an operand read (16 consecutive tokens of one unit) hits
// 16 distinct 16-byte bank groups, and one load instruction of a wave fills
// 1 KiB of the stage (4 tokens).  Weights run two chunks ahead in three
// register sets; the operand reads of step t + 1 are issued before the MFMAs
// of step t.  The stages are separate LDS arrays indexed statically (the
// chunk loop unrolls by six), so the compiler can tell that a load into one
// stage does not touch the other and does not wait for it before reading
// the other.  Several 4-wave workgroups share a CU (MB = 2: 33 KB of LDS
// and 164 VGPRs each), so each SIMD runs waves whose barriers are
// independent.
// (Measured at 16,384 tokens, config-4 FFN, median of 20 interleaved
// launches, the first form of this kernel -- MB = 4, 128-token tiles, two
// workgroups per CU: gate|up 466.7 us, down 225.6 us, against the
// token-half form it replaced, 556.4 and 244.8; 64-token tiles then measured equal
// or faster at every size (the launcher's sweep).  Rejected variants: one
// 8-wave workgroup of 512 rows per CU, 524.1 and 252.3; three stages,
// activations two chunks ahead, 656.5 / 280.5 with 4 waves (one workgroup
// per CU) and 534.8 / 254.7 with 8; persistent workgroups that issue the
// next tile's first loads before the epilogue, 699 with 4 waves (the tile
// loop spills).)
// s_waitcnt vmcnt(n) lgkmcnt(0) (expcnt at its maximum: no wait)
#define TW_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (0x7 << 4) | (((n) >> 4) << 14))
// a compiler-level fence: no memory operation moves across it
#define TW_ORDER() asm volatile("" ::: "memory")

template <int EPI, bool TILED = false, int MB = 4, bool SPLIT = false>
__global__ __launch_bounds__(256, 2) void k_tgemm_w(GemmArgs a) {
  constexpr int WR = 4, NB = 2, MT = 32 * MB;  // MT tokens per workgroup
  constexpr int STAGE = MT * TG_KC;
  constexpr int PI = STAGE / 1024 / WR;  // 1 KiB stage loads per wave and chunk
  constexpr int NWL = 2 * NB;               // weight load instructions per wave and chunk
  typedef uint32_t wvec __attribute__((ext_vector_type(8 * NB)));
  __shared__ __align__(1024) uint8_t s_a0[STAGE];
  __shared__ __align__(1024) uint8_t s_a1[STAGE];
  __shared__ float s_gm[128];
  __shared__ int32_t s_tp[EPI == NLG_EPI_QKV ? 128 : 1];
  __shared__ uint64_t s_tb[EPI == NLG_EPI_QKV ? 128 : 1];
  asm volatile("" ::"s"(a.xq), "s"(a.gamma), "s"(a.w2), "s"(a.bias), "s"(a.beta), "s"(a.y), "s"(a.seq),
               "s"(a.out), "s"(a.cols), "s"(a.wng), "s"(a.ystride), "s"(a.beta_per_row));
  const int lane = threadIdx.x & 63;
  const int wn = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, lg = lane >> 5;
  const uint32_t rbase = blockIdx.x * (64 * WR) + wn * 64;
  const uint32_t tok0 = blockIdx.y * MT;
  // SPLIT: slice blockIdx.z of gridDim.z takes chunks cfirst .. + nchunks - 1
  const uint32_t ntot = a.cols / TG_KC, ks = SPLIT ? gridDim.z : 1;
  const uint32_t cfirst = SPLIT ? blockIdx.z * ntot / ks : 0;
  const uint32_t nchunks = SPLIT ? (blockIdx.z + 1) * ntot / ks - cfirst : ntot;
  // weight rows of this lane: lane group lg holds words 8 lg .. 8 lg + 7 of
  // each chunk of rows rw[nt] (the tiled copy stores them in that order)
  uint32_t rw[NB], rc[NB];
  const uint4 *wp[NB];
#pragma unroll
  for (int nt = 0; nt < NB; nt++) {
    rw[nt] = rbase + 32 * nt + li;
    rc[nt] = rw[nt] < a.out ? rw[nt] : a.out - 1;
    if (TILED) {
      const uint32_t nrb = (a.out + 31) / 32, rb = rbase / 32 + nt < nrb ? rbase / 32 + nt : nrb - 1;
      wp[nt] = (const uint4 *)a.w2 + ((size_t)rb * ntot + cfirst) * 128 + lane;
    } else {
      wp[nt] = (const uint4 *)(a.w2 + (size_t)rc[nt] * a.wng) + 2 * lg + 4 * cfirst;
    }
  }
  // Stage loads: wave wn's load i fills stage bytes [1024 b, 1024 b + 1024),
  // b = wn PI + i: lane j writes token k = 4 b + j / 16 (clamped to the last
  // real token), slot j % 16, i.e. unit (j % 16) ^ (k % 16) of its chunk row,
  // at byte offset xo[i] from column 0 of the workgroup's first token row
  // (under MT x 16384 bytes: the loads take a scalar base + 32-bit offset)
  uint32_t xo[PI];
#pragma unroll
  for (int i = 0; i < PI; i++) {
    const uint32_t k = 4 * (wn * PI + i) + lane / 16, tk = tok0 + k < a.seq ? tok0 + k : a.seq - 1;
    xo[i] = (tk - tok0) * a.cols + 16 * ((lane % 16) ^ (k % 16));
  }
  const uint8_t *const xrow0 = a.xq + (size_t)tok0 * a.cols + (size_t)cfirst * TG_KC;
#define TW_LOADW(c, dst)                                                                   \
  do {                                                                                     \
    _Pragma("unroll") for (int nt = 0; nt < NB; nt++) {                                    \
      const uint4 u0 = TILED ? wp[nt][128 * (c)] : wp[nt][4 * (c)];                         \
      const uint4 u1 = TILED ? wp[nt][128 * (c) + 64] : wp[nt][4 * (c) + 1];                \
      dst[8 * nt + 0] = u0.x; dst[8 * nt + 1] = u0.y; dst[8 * nt + 2] = u0.z;               \
      dst[8 * nt + 3] = u0.w; dst[8 * nt + 4] = u1.x; dst[8 * nt + 5] = u1.y;               \
      dst[8 * nt + 6] = u1.z; dst[8 * nt + 7] = u1.w;                                       \
    }                                                                                      \
  } while (0)
#define TW_LOADA(c, stage)                                                                 \
  do {                                                                                     \
    const uint8_t *xc = xrow0 + (size_t)(c) * TG_KC;                                       \
    _Pragma("unroll") for (int i = 0; i < PI; i++)                                         \
      __builtin_amdgcn_global_load_lds(                                                    \
          (const void *)(xc + xo[i]),                                                      \
          (__attribute__((address_space(3))) void *)((stage) + 1024 * (wn * PI + i)), 16, 0, 0); \
  } while (0)
  // the epilogue operands first (their loads precede every stage load, so
  // they do not enter the waits' counts), then the first chunks in the order
  // the steps issue theirs: stage loads, then weight loads
  float bo[NB], be[NB];
#pragma unroll
  for (int nt = 0; nt < NB; nt++) {
    bo[nt] = a.bias ? a.bias[rc[nt]] : 0.0f;
    be[nt] = a.beta[a.beta_per_row ? rc[nt] : 0];
  }
  const uint32_t tkc = tok0 + threadIdx.x % MT < a.seq ? tok0 + threadIdx.x % MT : a.seq - 1;
  const float gm_r = a.gamma[tkc];
  int32_t tp_r = 0;
  uint64_t tb_r = 0;
  if (EPI == NLG_EPI_QKV) {
    // token t's cache position (decode rows: pos[0]; prompt rows: pos[0] +
    // t % qper) and its cache row's element offset
    const int32_t pr = nlg_ld_uniform_i32(a.pos) + (a.qper ? (int32_t)(tkc % a.qper) : 0);
    const bool ok = pr >= 0 && (uint32_t)pr < a.max_seq;
    const uint32_t sq = a.qper ? tkc / a.qper : tkc;
    tp_r = ok ? pr : -1;
    tb_r = ((uint64_t)sq * a.kvheads * a.max_seq + (ok ? (uint32_t)pr : 0u)) * a.hd;
  }
  wvec wA, wB, wC;
  const uint32_t c1 = nchunks > 1 ? 1 : 0;
  TW_ORDER();
  TW_LOADW(0, wA);
  TW_ORDER();
  TW_LOADA(0, s_a0);
  TW_ORDER();
  TW_LOADW(c1, wB);
  // (stored before the first step, whose wait includes lgkmcnt(0))
  if (threadIdx.x < MT) {
    s_gm[threadIdx.x] = gm_r;
    if (EPI == NLG_EPI_QKV) {
      s_tp[threadIdx.x] = tp_r;
      s_tb[threadIdx.x] = tb_r;
    }
  }
  v16i acc[MB][NB];  // [token block][row block]
#pragma unroll
  for (int mt = 0; mt < MB; mt++)
#pragma unroll
    for (int nt = 0; nt < NB; nt++) acc[mt][nt] = (v16i){};
  // the operand read of lane (li, lg), token block mt, step t: token
  // k = 32 mt + li, unit 8 lg + t, at k * 256 + 16 ((8 lg + t) ^ (li % 16))
  const uint32_t ra = li * TG_KC + 16 * ((8 * lg) ^ (li % 16));
#define TW_RDA(stage, t, dst)                                                                 \
  do {                                                                                        \
    const uint8_t *sp = (stage) + (ra ^ (16 * (t)));                                          \
    _Pragma("unroll") for (int mt = 0; mt < MB; mt++) {                                       \
      const uint4 u = *(const uint4 *)(sp + 32 * TG_KC * mt);                                  \
      dst[mt] = (v4i){(int)u.x, (int)u.y, (int)u.z, (int)u.w};                                 \
    }                                                                                         \
  } while (0)
  // each A fragment feeds NB MFMAs, each decoded B operand MB
#define TW_MMA(stage, WCUR)                                                                   \
  {                                                                                           \
    v4i av[2][MB];                                                                            \
    TW_RDA(stage, 0, av[0]);                                                                  \
    _Pragma("unroll") for (int t = 0; t < 8; t++) {                                           \
      if (t < 7) TW_RDA(stage, t + 1, av[(t + 1) & 1]);                                       \
      __builtin_amdgcn_sched_barrier(0);                                                      \
      _Pragma("unroll") for (int nt = 0; nt < NB; nt++) {                                     \
        const uint32_t x0 = WCUR[8 * nt + t];                                                 \
        const v4i b0 = {(int)((x0 << 6) & 0xC0C0C0C0u), (int)((x0 << 4) & 0xC0C0C0C0u),       \
                        (int)((x0 << 2) & 0xC0C0C0C0u), (int)(x0 & 0xC0C0C0C0u)};              \
        _Pragma("unroll") for (int mt = 0; mt < MB; mt++)                                     \
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[t & 1][mt], b0, acc[mt][nt], 0, 0, 0); \
      }                                                                                       \
    }                                                                                         \
  }
  // chunk c (stage SCUR, weights WCUR): wait for this wave's loads of chunk
  // c's stage (a step issues its stage loads, then its NWL weight loads, so
  // only the previous step's weight loads -- chunk c + 1's -- may still be
  // out), meet the workgroup (every stage load of chunk c has landed; every
  // wave is done reading SLOAD, chunk c - 1's stage), load chunk c + 1's
  // activations into SLOAD and chunk c + 2's weights into WLOAD (clamped:
  // the last fetches repeat), multiply chunk c
#define TW_STEP(k, SCUR, SLOAD, WCUR, WLOAD)                                                  \
  {                                                                                           \
    const uint32_t c = c0 + (k);                                                              \
    TW_ORDER();                                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                        \
    TW_WAIT_VM(NWL);                                                                          \
    __builtin_amdgcn_s_barrier();                                                             \
    TW_ORDER();                                                                               \
    TW_LOADA(c + 1 < nchunks ? c + 1 : nchunks - 1, SLOAD);                                   \
    TW_ORDER();                                                                               \
    TW_LOADW(c + 2 < nchunks ? c + 2 : nchunks - 1, WLOAD);                                   \
    __builtin_amdgcn_sched_barrier(0);                                                        \
    TW_MMA(SCUR, WCUR);                                                                       \
  }
  // whole groups of six chunks (stages alternate, weight sets rotate by
  // three), then up to five, nested so that no register set is merged at a
  // join
  uint32_t c0 = 0;
  for (; c0 + 6 <= nchunks; c0 += 6) {
    TW_STEP(0, s_a0, s_a1, wA, wC)
    TW_STEP(1, s_a1, s_a0, wB, wA)
    TW_STEP(2, s_a0, s_a1, wC, wB)
    TW_STEP(3, s_a1, s_a0, wA, wC)
    TW_STEP(4, s_a0, s_a1, wB, wA)
    TW_STEP(5, s_a1, s_a0, wC, wB)
  }
  if (c0 < nchunks) {
    TW_STEP(0, s_a0, s_a1, wA, wC)
    if (c0 + 1 < nchunks) {
      TW_STEP(1, s_a1, s_a0, wB, wA)
      if (c0 + 2 < nchunks) {
        TW_STEP(2, s_a0, s_a1, wC, wB)
        if (c0 + 3 < nchunks) {
          TW_STEP(3, s_a1, s_a0, wA, wC)
          if (c0 + 4 < nchunks) TW_STEP(4, s_a0, s_a1, wB, wA)
        }
      }
    }
  }
#undef TW_STEP
#undef TW_MMA
#undef TW_RDA
#undef TW_LOADW
#undef TW_LOADA
  // the last (repeated) stage loads must land before the workgroup's LDS is
  // released
  TW_WAIT_VM(0);
  if (SPLIT) {
    __shared__ uint32_t s_last;
    if (!tl_split_meet<MB, NB>(a, acc, &s_last)) return;
  }
  tl_epilogue<MB, NB, EPI>(a, acc, rw, rc, bo, be, s_gm, lane, 0, lg, tok0, s_tp, s_tb);
}
#undef TW_ORDER
#undef TW_WAIT_VM

// ------------------------------------------------------------ launchers

int nlg_act_q_launch(const float *x, const float *gain, float eps, const float *attn_mz, uint32_t attn_nc,
                     uint32_t hd, int pro, uint8_t *xq, float *gamma, uint32_t seq, uint32_t cols,
                     hipStream_t st) {
  if (!seq) return NLG_OK;
  if (cols % 64 || !cols || cols > 16384) return nlg_fail("act quant: cols must be a multiple of 64 in [64, 16384]");
  ActQArgs a{x, gain, eps, attn_mz, attn_nc, hd, xq, gamma, seq, cols, seq >= 2048u};
  const dim3 grid(seq), blk(256);
#define AQ(P)                                                                                      \
  do {                                                                                             \
    if (cols <= 4096) hipLaunchKernelGGL((k_act_q<1, P>), grid, blk, 0, st, a);                    \
    else if (cols <= 8192) hipLaunchKernelGGL((k_act_q<2, P>), grid, blk, 0, st, a);               \
    else hipLaunchKernelGGL((k_act_q<4, P>), grid, blk, 0, st, a);                                 \
  } while (0)
  if (pro == NLG_PRO_RMS) AQ(NLG_PRO_RMS);
  else if (pro == NLG_PRO_ATTN && attn_nc == 3) AQ(NLG_PRO_ATTN3);
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
  // a registered tiled copy of the weights (nlg_ternary_tiled_register)
  // replaces the row layout: the same words, in load order
  const uint32_t *wt = nlg_tiled_find(a.w2, a.out, a.cols);
  if (wt) a.w2 = wt;
  // Rows of 9..10 chunks over 128..256 64-row x 32-token tiles take
  // k_tgemm's single 10-chunk phase below at any token count: at 128..192
  // tokens (QKV 3,840 rows at 128, O 2,560 rows up to 192) it beat the
  // wide-wave kernel's 32-token tiles 6.2..6.4 against 10.2..10.4 us, while
  // its two-phase forms (more tiles) lost or tied.
  const uint32_t nch_all = a.cols / TG_KC;
  const uint64_t t64x32 = (uint64_t)nlg_blocks(a.out, 64) * ((a.seq + 31) / 32);
  const bool one_phase = nch_all > TG_PH && nch_all <= 10 && t64x32 >= 128 && t64x32 <= 256;
  // From 65 tokens, more than 512 such tiles (k_tgemm holds two 64-row
  // workgroups per CU, so a second round) go to the wide-wave kernel too:
  // gate|up (13,824 x 2560) at 72 / 96 / 112 / 127 tokens 12.8 / 12.4 /
  // 12.5 / 13.9 against 15.8 / 16.2 / 19.6 / 19.9 us, 13,824 x 1280 at 72
  // 8.7 against 9.6; at 432 tiles k_tgemm kept the lead (gate|up at 64
  // tokens 10.9 against 11.7, 6,912 x 2560 at 112 10.6 against 12.0).
  const bool wide = a.seq >= 128 || (a.seq > 64 && t64x32 > 512);
  if (wide && epi != NLG_EPI_ARGMAX && !one_phase) {
    // 256-row tiles of the wide-wave kernel (k_tgemm_w), 64-token tiles
    // once there are 400 of them, else 32-token ones; a few tiles of long
    // rows split their columns over gridDim.z slices.  From sweeps of the
    // config-5 linears and config 4 at 128..16384 tokens, kernel trace,
    // median of 6..20 interleaved launches of each form:
    //  * 32-token tiles against the token-half 64-row-tile form this kernel
    //    replaced, tiled weights, residual epilogue: QKV at 128 / 256 / 512 /
    //    1024 tokens 11.6 / 11.4 / 13.5 / 17.5 us against 13.6 / 14.9 / 16.0
    //    / 22.2; O 11.0 / 10.8 / 12.0 / 16.0 against 12.8 / 13.8 / 15.4 /
    //    19.5; down at 1024 30.1 against 39.3; gate|up at 128 / 256 12.1 /
    //    17.8 against 14.5 / 22.4.
    //  * 64-token tiles against 32-token ones: gate|up at 512 / 1024 / 2048 /
    //    4096 / 16384 tokens (432..13824 tiles) 26.0 / 51.4 / 99.4 / 176.2 /
    //    743 against 27.0 / 52.2 / 106.6 / 196.9 / 808; QKV at 2048 / 4096
    //    (480 / 960) 27.4 / 50.7 against 28.1 / 52.6; but O and down at 2048
    //    (320) 24.5 / 47.4 against 21.6 / 43.2, QKV at 1024 (240) 19.8
    //    against 17.5.
    //  * 128-token tiles (4 token blocks per wave, two workgroups per CU)
    //    against 64-token ones, same epilogues as config 4: gate|up (SwiGLU)
    //    at 1024 / 2048 / 4096 / 16384 tokens 40.3 / 75.6 / 156.5 / 550.4
    //    against 40.2 / 68.9 / 150.2 / 550.0, down (STORE) 49.8 / 54.7 /
    //    102.1 / 265.3 against 29.8 / 44.8 / 81.9 / 251.5: not kept.
    //  * the column split of 32-token tiles, 2 / 3 / 4 slices against none,
    //    tiled weights (row layout within 1 us of these): down projection
    //    (2560 x 6912, 27 chunks) at 128 tokens (40 tiles) 15.0 / 14.3 /
    //    14.4 against 19.4, 256 (80) 15.9 / 15.1 / 17.7 against 19.6, 384
    //    (120) 17.2 / 19.2 / 18.2 against 20.0, 512 (160) 22.6 / 20.0 / 22.7
    //    against 21.0, 640 (200) 23.2 / 24.9 / 26.1 against 21.5; 1024 x 6912
    //    at 128 (16) 15.0 / 14.3 / 13.3 against 18.5; 2560 x 4096 at 128 (40)
    //    12.8 / 12.1 / 12.5 against 14.2; but rows of 10 chunks never gain
    //    (O 2560 x 2560 at 128 / 256 / 512 tokens 10.3 / 10.5 / 11.9 unsplit,
    //    10.9 / 11.8 / 15.3 in 2 slices; QKV 3840 x 2560 likewise).  The
    //    split form the kernel replaced (64-row tiles of token-half waves)
    //    took 16.2 / 20.0 / 20.5 us for the down projection at 128 / 256 /
    //    384 tokens.  Every slice leaves a 32 KB block of partial sums and
    //    the last to arrive reads the others (tl_split_meet), so a slice
    //    must carry enough chunks: rows of 16+ chunks only, and about one
    //    workgroup per CU in all (two at 160 tiles).
    const uint32_t rt = nlg_blocks(a.out, 256);
    const uint64_t n32 = (a.seq + 31) / 32, t1 = (uint64_t)rt * n32, t2 = (uint64_t)rt * ((a.seq + 63) / 64);
    const uint32_t nch = a.cols / TG_KC;
    uint32_t ks = 1;
    if (a.allow_split && nch >= 16) {
      if (t1 <= 128) ks = 256 / (uint32_t)t1 < 4 ? 256 / (uint32_t)t1 : 4;  // >= 2
      else if (t1 <= 170) ks = 3;
    }
    if (ks > 1) {
      // partial sums: one 32-register block per (slice, tile, thread); the
      // counters' region is the same for every launch (a split grid has at
      // most 170 tiles), so partial sums never land on a counter
      const size_t ctr_bytes = 256 * 4;
      uint8_t *w = (uint8_t *)nlg_scratch_try(ctr_bytes + (size_t)ks * t1 * 256 * 32 * 4, st, 1);
      if (w) {
        a.kctr = (uint32_t *)w;
        a.ksum = (int32_t *)(w + ctr_bytes);
      } else {
        ks = 1;
      }
    }
    const bool t64 = ks == 1 && t2 >= 400;
    const dim3 gw(rt, t64 ? (a.seq + 63) / 64 : (uint32_t)n32, ks);
    if (gw.y > 65535) return nlg_fail("ternary GEMM: seq too large");
#define TWT(E, T)                                                                                \
  do {                                                                                           \
    if (ks > 1) hipLaunchKernelGGL((k_tgemm_w<E, T, 1, true>), gw, dim3(256), 0, st, a);         \
    else if (t64) hipLaunchKernelGGL((k_tgemm_w<E, T, 2>), gw, dim3(256), 0, st, a);            \
    else hipLaunchKernelGGL((k_tgemm_w<E, T, 1>), gw, dim3(256), 0, st, a);                     \
  } while (0)
#define TWG(E)                                                                                   \
  do {                                                                                           \
    if (wt) TWT(E, true);                                                                        \
    else TWT(E, false);                                                                          \
  } while (0)
    switch (epi) {
      case NLG_EPI_STORE: TWG(NLG_EPI_STORE); break;
      case NLG_EPI_RESID: TWG(NLG_EPI_RESID); break;
      case NLG_EPI_SWIGLU: TWG(NLG_EPI_SWIGLU); break;
      case NLG_EPI_QKV: TWG(NLG_EPI_QKV); break;
      default: return nlg_fail("ternary GEMM: unknown epilogue %d", epi);
    }
#undef TWG
#undef TWT
    NLG_LAUNCHED(ks > 1 ? "ternary GEMM (int8 MFMA, wide waves, column split)" : "ternary GEMM (int8 MFMA, wide waves)");
    return NLG_OK;
  }
  // up to 32 tokens per workgroup: the 32 x 2064-byte activation block
  // stays under the 64 KiB a workgroup may hold
  const int MB = a.seq <= 16 ? 1 : 2;
  const uint32_t MT = 16u * MB;
  if (epi != NLG_EPI_ARGMAX && (uint64_t)nlg_blocks(a.out, 64) * ((a.seq + MT - 1) / MT) < 128) {
    // too few 64-row workgroups to fill half the CUs: 16-row ones with the
    // columns split over the waves (measured at 32 tokens: 2560..3840 rows
    // gain, 13,824 rows lose to the extra activation reads), of 16 tokens up
    // to 32 (each workgroup reads its token block of every chunk, 8x its
    // weight bytes at 16 rows; twice the workgroups with half the block:
    // B=32 decode QKV 8.44 -> 7.55 us, O with its merge 8.11 -> 7.66, down
    // 9.88 -> 9.99, 19.9k -> 20.1k tok/s; k_tgemm's 64-row gate|up lost
    // 1.0 us to the same change and keeps 32-token workgroups)
    const int MBK = a.seq <= 32 ? 1 : 2;
    const uint32_t MTK = 16u * MBK;
    const dim3 grid(nlg_blocks(a.out, 16), (a.seq + MTK - 1) / MTK), blk(256);
    if (grid.y > 65535) return nlg_fail("ternary GEMM: seq too large");
    // weight chunks per wave: the smallest instantiated count >= ceil(chunks / 4)
    const uint32_t per = (a.cols / TG_KC + 3) / 4;
    const int pm = per <= 2 ? 2 : per <= 3 ? 3 : per <= 4 ? 4 : per <= 7 ? 7 : 16;
#define TKT(M, E, T)                                                                      \
  do {                                                                                    \
    if (pm == 2) hipLaunchKernelGGL((k_tgemm_k<M, E, 2, T>), grid, blk, 0, st, a);        \
    else if (pm == 3) hipLaunchKernelGGL((k_tgemm_k<M, E, 3, T>), grid, blk, 0, st, a);   \
    else if (pm == 4) hipLaunchKernelGGL((k_tgemm_k<M, E, 4, T>), grid, blk, 0, st, a);   \
    else if (pm == 7) hipLaunchKernelGGL((k_tgemm_k<M, E, 7, T>), grid, blk, 0, st, a);   \
    else hipLaunchKernelGGL((k_tgemm_k<M, E, 16, T>), grid, blk, 0, st, a);               \
  } while (0)
#define TKP(M, E)                                                                         \
  do {                                                                                    \
    if (wt) TKT(M, E, true);                                                              \
    else TKT(M, E, false);                                                                \
  } while (0)
#define TKG(E)                                                                            \
  do {                                                                                    \
    if (MBK == 1) TKP(1, E);                                                              \
    else TKP(2, E);                                                                       \
  } while (0)
    switch (epi) {
      case NLG_EPI_STORE: TKG(NLG_EPI_STORE); break;
      case NLG_EPI_RESID: TKG(NLG_EPI_RESID); break;
      case NLG_EPI_SWIGLU: TKG(NLG_EPI_SWIGLU); break;
      case NLG_EPI_QKV: TKG(NLG_EPI_QKV); break;
      default: return nlg_fail("ternary GEMM: unknown epilogue %d", epi);
    }
#undef TKG
#undef TKP
#undef TKT
    NLG_LAUNCHED("ternary GEMM (int8 MFMA, split columns)");
    return NLG_OK;
  }
  const dim3 grid(nlg_blocks(a.out, 64), (a.seq + MT - 1) / MT), blk(256);
  if (grid.y > 65535) return nlg_fail("ternary GEMM: seq too large");
  if (epi == NLG_EPI_ARGMAX) a.nparts = grid.x;
  const uint32_t nch = a.cols / TG_KC;
  if ((epi == NLG_EPI_ARGMAX || epi == NLG_EPI_STORE) && (uint64_t)grid.x * grid.y >= 1024) {
    // Many 64-row tiles of few tokens (the LM head): the wide-wave kernel in
    // 32-token tiles (each wave 64 rows, one weight fetch per tile, the
    // argmax partial of its 64 rows where k_tgemm's workgroup would put it).
    // Measured on the 128,256 x 2,560 LM head with its quantisation and
    // argmax launches, tiled weights, graph-replayed: 32 tokens 41.8 ->
    // 33.9 us, 8 tokens 30.5 -> 28.4, against the form it replaced (one
    // 8-wave workgroup per CU staging its token block once and walking
    // 128-row tiles of 16-row waves: every wave re-read the whole block from
    // LDS for each tile); that form had replaced k_tgemm's 64-row tiles at
    // 63.2 -> 49.3 us for 32 tokens.
    const dim3 gw(nlg_blocks(a.out, 256), (a.seq + 31) / 32);
#define TWR(E)                                                                                   \
  do {                                                                                           \
    if (wt) hipLaunchKernelGGL((k_tgemm_w<E, true, 1>), gw, dim3(256), 0, st, a);              \
    else hipLaunchKernelGGL((k_tgemm_w<E, false, 1>), gw, dim3(256), 0, st, a);                \
  } while (0)
    if (epi == NLG_EPI_ARGMAX) TWR(NLG_EPI_ARGMAX);
    else TWR(NLG_EPI_STORE);
#undef TWR
    NLG_LAUNCHED("ternary GEMM (int8 MFMA, wide waves)");
    return NLG_OK;
  }
  // Rows of 9..10 chunks (2560 columns) take one 10-chunk phase, one memory
  // round trip instead of two, when the grid is a single round of workgroups
  // (its 82 KB stage admits one per CU)
  const bool ph10 = nch > TG_PH && nch <= 10 && (uint64_t)grid.x * grid.y <= 256;
  const size_t lds = (size_t)MT * (ph10 ? 10 * TG_KC + 16 : TG_PITCH);
  const int nph = a.cols <= 2048 ? 1 : (a.cols <= 4096 ? 2 : (a.cols <= 8192 ? 4 : 8));
#define TGT(M, E, T)                                                                              \
  do {                                                                                            \
    if (ph10) hipLaunchKernelGGL((k_tgemm<M, 1, 10, E, T>), grid, blk, lds, st, a);               \
    else if (nph == 1) hipLaunchKernelGGL((k_tgemm<M, 1, TG_PH, E, T>), grid, blk, lds, st, a);   \
    else if (nph == 2) hipLaunchKernelGGL((k_tgemm<M, 2, TG_PH, E, T>), grid, blk, lds, st, a);   \
    else if (nph == 4) hipLaunchKernelGGL((k_tgemm<M, 4, TG_PH, E, T>), grid, blk, lds, st, a);   \
    else hipLaunchKernelGGL((k_tgemm<M, 8, TG_PH, E, T>), grid, blk, lds, st, a);                 \
  } while (0)
#define TGP(M, E)                                                                                 \
  do {                                                                                            \
    if (wt) TGT(M, E, true);                                                                      \
    else TGT(M, E, false);                                                                        \
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
#undef TGT
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
  return nlg_batched_gemm(f, xq, gamma, epi, st);
}

int nlg_batched_gemm(const FusedArgs &f, const uint8_t *xq, const float *gamma, int epi, hipStream_t st) {
  GemmArgs g{};
  g.xq = xq; g.gamma = gamma; g.w2 = f.w2; g.bias = f.bias; g.beta = f.beta; g.beta_per_row = f.beta_per_row;
  g.seq = f.seq; g.out = f.out; g.cols = f.cols; g.y = f.y; g.ystride = f.ystride; g.res = f.res;
  g.rstride = f.rstride; g.nq = f.nq; g.nkv = f.nkv; g.hd = f.hd; g.kvheads = f.kvheads; g.max_seq = f.max_seq;
  g.co = f.co; g.si = f.si; g.pos = f.pos; g.kc = f.kc; g.vc = f.vc; g.qper = f.qper;
  g.pval = f.pval; g.pidx = f.pidx;
  g.allow_split = !f.act_scratch;  // caller-provided scratch: no library allocation
  return nlg_tgemm_launch(g, epi, st);
}
