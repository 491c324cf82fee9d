// nlg_layer.hip -- the decoder layer's fused kernels.
//
// k_tern_fused: one launch per ternary linear of a decode step.  Each
// workgroup (4 waves, R output rows per wave) issues its weight loads first,
// then -- while they are in flight -- optionally RMS-normalises the token's
// activation row, quantises it exactly as pack-act-rows does into LDS, dots
// its rows against it, and finishes with one of these epilogues:
//
//   STORE   Y = BIAS + (BETA*GAMMA)*acc            bitlinear-dp4a-1f (kernels.el:619-634)
//   RESID   X = X + that                           add2 (kernels.el:812-821)
//   SWIGLU  rows 2j/2j+1 are gate/up row j:        silu-mul (kernels.el:186-193)
//           H[j] = (g * 1/(1+exp(0-g))) * u
//   QKV     rows are q | k | v: RoPE on q and k    decode-rope(-b) (kernels.el:291-306, :340-355)
//           at the device position, k and v        cache-append(-b) (kernels.el:307-314, :356-365)
//           appended to fp16 caches
//   ARGMAX  logits, plus (max, first index) per wave for greedy sampling
//
// The RMSNorm prologue is rmsnorm-istd + rmsnorm-fwd (kernels.el:1249-1265)
// with the epsilon a parameter: S = 1/sqrt(sum(x*x)/N + eps), C = (X*S)*G.
// Its sum is a tree, not the reference's serial loop, so S can differ from
// the reference in the last bit; everything after it is the reference's
// arithmetic.

// The fp16 decode attention these layers feed lives in nlg_dattn.hip.
#include <math.h>

#include "nlg_quant.h"

// ------------------------------------------------------------ fused GEMV

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);  // round to nearest even
}

// F4: float4s of the activation row per thread (cols <= 1024*F4).
template <int R, int CPL, int F4, int PRO, int EPI>
__global__ __launch_bounds__(256) void k_tern_fused(FusedArgs a) {
  extern __shared__ uint4 s_xq4[];  // 64 F4 uint4: cols int8 lanes, then the words past the row
  __shared__ float red[4], red2[4];  // the two reductions' own scratch: no reuse barrier
  // Every argument the kernel uses is pinned into SGPRs here, so they all
  // arrive with the first kernarg fetch instead of in later round trips.
  // TIMED: the wave's start on the constant 100 MHz wall clock (a scalar
  // read of the clock, no memory access); its end is taken after its stores
  constexpr bool TIMED = EPI == NLG_EPI_STORE_TIMED;
  const unsigned long long t_start = TIMED ? __builtin_amdgcn_s_memrealtime() : 0ull;
  float *const y_out = a.y;
  float *const gamma_out = a.gamma_out;
  const uint32_t ystride = a.ystride;
  asm volatile("" ::"s"(y_out), "s"(gamma_out), "s"(ystride));
  // the wave index as a scalar: row addresses then live in SGPRs and each
  // load is one SGPR base plus the lane's offset (no 64-bit vector math
  // ahead of the weight stream)
  const int lane = threadIdx.x & 63, wvi = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t tok = blockIdx.y;
  const uint32_t wave = blockIdx.x * 4 + wvi;
  const uint32_t row0 = wave * R;
  const uint32_t nchunk = a.wng >> 2;
  // 1. every global load is issued up front, activation first: vmcnt retires
  //    in issue order, so waiting for x must not also wait for the weights'
  //    HBM fetch, which stays in flight through the quantisation below.  The
  //    loads are straight-line (clamped addresses, validity applied with
  //    selects afterwards): a branch around a load makes the wait-count pass
  //    drain every outstanding load at the join.
  // QKV: the device position, as a scalar load (a vector load of it, issued
  // behind the weights, made the RoPE lookup wait for their HBM fetch)
  int32_t pos0 = 0;
  if (EPI == NLG_EPI_QKV) pos0 = nlg_ld_uniform_i32(a.pos);
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t nf4 = a.cols >> 2;
  float4 xv4[F4], gv4[F4];
  // PRO_ATTN: the chunk contexts and (max, sum) pairs of every element
  // (PRO_ATTN3: exactly three chunks, so no clamped repeat of the last one
  // is loaded; the fourth chunk's weight is 0 in the general form, so the
  // merged values differ at most in the sign of a zero, which quantises alike)
  constexpr bool ATT = PRO == NLG_PRO_ATTN || PRO == NLG_PRO_ATTN3;
  // PRO_NONE: the activation is loaded already transposed (below).  The
  // RMS and merge prologues keep float4 loads: their sums run in the batched
  // quantiser's element order, so both forms quantise a row alike.
  constexpr bool XPOSE_LOAD = PRO == NLG_PRO_NONE;
  constexpr int NCA = PRO == NLG_PRO_ATTN3 ? 3 : (ATT ? NLG_ATTN_MAX_CHUNKS : 1);
  float4 cx4[F4][NCA];
  float2 mz2[F4][NCA];
  if (ATT) {
    const float4 *c4 = (const float4 *)a.x;
    const uint32_t heads = a.cols / a.hd;
#pragma unroll
    for (int k = 0; k < F4; k++) {
      const uint32_t f = threadIdx.x + 256u * k, fc = f < nf4 ? f : nf4 - 1;
      const uint32_t h = (4 * fc) / a.hd;
#pragma unroll
      for (int c = 0; c < NCA; c++) {
        const uint32_t cc = (uint32_t)c < a.attn_nc ? (uint32_t)c : a.attn_nc - 1;
        const size_t tc = (size_t)tok * a.attn_nc + cc;
        cx4[k][c] = c4[tc * nf4 + fc];
        mz2[k][c] = *(const float2 *)(a.attn_mz + (tc * heads + h) * 2);
      }
    }
  } else if (XPOSE_LOAD) {
    // word f of the LDS row is byte i of the four words of its 16-column
    // group (the dots' operand order), i.e. columns 16 (f / 4) + f % 4 + 4 m,
    // m = 0..3: loaded in that order, the quantised bytes pack straight into
    // it (no cross-lane transpose); the quad's four loads of a 16-column
    // group read one 64-byte piece.  Buffer loads bounded by the row: words
    // past it read 0 (no clamped addresses, one offset register for all)
    const __amdgpu_buffer_rsrc_t xr = nlg_buffer_rsrc(a.x + (size_t)tok * a.cols, a.cols * 4u);
    const int32_t xo = (int32_t)(4u * (16u * (threadIdx.x >> 2) + (threadIdx.x & 3u)));
#pragma unroll
    for (int k = 0; k < F4; k++)
      xv4[k] = make_float4(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, xo, 4096 * k, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, xo + 16, 4096 * k, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, xo + 32, 4096 * k, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, xo + 48, 4096 * k, 0)));
  } else {
    const float4 *x4 = (const float4 *)(a.x + (size_t)tok * a.cols);
#pragma unroll
    for (int k = 0; k < F4; k++) {
      const uint32_t f = threadIdx.x + 256u * k;
      xv4[k] = x4[f < nf4 ? f : nf4 - 1];
    }
  }
  if (PRO == NLG_PRO_RMS) {
    const float4 *g4 = (const float4 *)a.gain;
#pragma unroll
    for (int k = 0; k < F4; k++) {
      const uint32_t f = threadIdx.x + 256u * k;
      gv4[k] = g4[f < nf4 ? f : nf4 - 1];
    }
  }
  // The epilogue's operands (a few bytes per row, cache-resident) before the
  // weight stream, which is issued last: nothing then waits behind it, and
  // its four loads go out back to back (with these after it, the 4096^2
  // step took 0.14 us longer).
  const uint32_t orow_u = row0 + (lane < R ? lane : 0);
  const uint32_t orow = orow_u < a.out ? orow_u : a.out - 1;  // every lane loads a valid row
  const bool olive = lane < R && orow_u < a.out;
  const float *bsrc = a.bias ? a.bias : a.beta;  // a real address either way
  constexpr bool PLAIN = EPI == NLG_EPI_STORE_PLAIN || EPI == NLG_EPI_STORE_TIMED;
  const float bo_raw = PLAIN ? 0.0f : bsrc[a.bias ? orow : 0];
  const float be = a.beta[PLAIN || !a.beta_per_row ? 0 : orow];
  const float bo = a.bias && !PLAIN ? bo_raw : 0.0f;
  float rv = 0.0f;
  if (EPI == NLG_EPI_RESID) rv = a.res[(size_t)tok * a.rstride + orow];
  // QKV: this lane's row is q, k or v; RoPE pair m of head dimension dd
  float cc = 0.0f, ss = 0.0f;
  uint32_t dd = 0, p = 0;
  bool pos_ok = false;
  if (EPI == NLG_EPI_QKV) {
    const int32_t pr = pos0 + (a.qper ? (int32_t)(tok % a.qper) : 0);
    pos_ok = pr >= 0 && (uint32_t)pr < a.max_seq;
    p = pos_ok ? (uint32_t)pr : 0u;
    const uint32_t sec = orow < a.nq ? orow : (orow < a.nq + a.nkv ? orow - a.nq : orow - a.nq - a.nkv);
    dd = sec % a.hd;
    const uint32_t half = a.hd >> 1, ci = p * half + (dd >> 1);
    cc = a.co[ci];
    ss = a.si[ci];  // SG[0] = +1: SI*SG is SI exactly
  }
  // Rows of at most 48 chunks (3072 columns: lanes 48..63 would idle on
  // every row) with R >= 4: G = 64/R lanes per row, lane (prow, pj)
  // holding chunks pj + G k of row row0 + prow in wv[k][0] -- every lane
  // busy and each row reduced over G lanes only.  Otherwise lane l holds
  // chunks l + 64 i of every row in wv[r][i] (at 4096 columns that reads
  // each activation chunk from LDS once per lane instead of R times; the
  // packed form there measured 3.48 -> 3.68 us for the 4096^2 step).
  constexpr bool PACK = CPL == 1 && F4 <= 3 && R >= 4;
  // packed rows: a row has at most 16 F4 chunks, so a lane holds at most
  // KPL = ceil(16 F4 / G) of them (3 of R = 4, 6 of 8, 12 of 16 at 2560
  // columns) -- no load issued for a chunk slot no row length can reach
  constexpr int G = PACK ? 64 / R : 64;
  const uint32_t prow = (uint32_t)lane / G, pj = (uint32_t)lane % G;
  constexpr int KPL = PACK ? ((16 * F4 + (64 / R) - 1) / (64 / R) < R ? (16 * F4 + (64 / R) - 1) / (64 / R) : R) : R;
  uint4 wv[R][CPL];
  if (PACK) {
    const uint32_t row = row0 + prow < a.out ? row0 + prow : a.out - 1;
    const uint4 *wr = (const uint4 *)(a.w2 + (size_t)row * a.wng);
#pragma unroll
    for (int k = 0; k < KPL; k++) {
      const uint32_t c = pj + G * k;
      wv[k][0] = nlg_ld_stream(&wr[c < nchunk ? c : nchunk - 1]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r < a.out ? row0 + r : a.out - 1;
      const uint4 *wr = (const uint4 *)(a.w2 + (size_t)row * a.wng);
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const uint32_t c = lane + 64 * i;
        wv[r][i] = nlg_ld_stream(&wr[c < nchunk ? c : nchunk - 1]);
      }
    }
  }
  // every load above issued before any of them is waited for
  __builtin_amdgcn_sched_barrier(0);
  // Chunks past the row stay as loaded (the dots skip them): writing a
  // register whose load is in flight waits for that load, which would put
  // the weights' HBM fetch in front of the quantisation.  Activation
  // float4s past the row (clamped repeats of the last one) change neither
  // the absmax nor any stored word, so only the RMS sum of squares needs
  // them zeroed -- by selects: a conditional block here made the wait-count
  // pass drain loads at its join (0.11 us of the 4096^2 step).
  if (PRO == NLG_PRO_RMS) {
#pragma unroll
    for (int k = 0; k < F4; k++) {
      const bool in = threadIdx.x + 256u * k < nf4;
      xv4[k] = make_float4(in ? xv4[k].x : 0.0f, in ? xv4[k].y : 0.0f, in ? xv4[k].z : 0.0f, in ? xv4[k].w : 0.0f);
    }
  }
  // 2a. attention merge: x = sum_c ctx_c*exp(m_c - M) / sum_c z_c*exp(m_c - M)
  //     in k_attn_merge's exact operation order, so the two agree bit for bit
  if (ATT) {
#pragma unroll
    for (int k = 0; k < F4; k++) {
      float mm = -1.0e30f;
#pragma unroll
      for (int c = 0; c < NCA; c++) mm = mz2[k][c].x > mm ? mz2[k][c].x : mm;
      float zz = 0.0f;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int c = 0; c < NCA; c++) {
        const float sc = (uint32_t)c < a.attn_nc ? nlg_exp2(mz2[k][c].x - mm) : 0.0f;  // base-2 maxima
        zz = fmaf(mz2[k][c].y, sc, zz);
        acc.x = fmaf(cx4[k][c].x, sc, acc.x);
        acc.y = fmaf(cx4[k][c].y, sc, acc.y);
        acc.z = fmaf(cx4[k][c].z, sc, acc.z);
        acc.w = fmaf(cx4[k][c].w, sc, acc.w);
      }
      xv4[k] = make_float4(acc.x / zz, acc.y / zz, acc.z / zz, acc.w / zz);
    }
  }
  // 2. RMSNorm: S = 1/sqrt(sum(x*x)/N + eps); C = (X*S)*G
  if (PRO == NLG_PRO_RMS) {
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < F4; k++) {
      sq = sq + xv4[k].x * xv4[k].x;
      sq = sq + xv4[k].y * xv4[k].y;
      sq = sq + xv4[k].z * xv4[k].z;
      sq = sq + xv4[k].w * xv4[k].w;
    }
    sq = nlg_block_sum_f32<4, true>(sq, red);
    sq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq)));
    const float istd = 1.0f / sqrtf(sq / (float)a.cols + a.eps);
#pragma unroll
    for (int k = 0; k < F4; k++) {
      xv4[k].x = (xv4[k].x * istd) * gv4[k].x;
      xv4[k].y = (xv4[k].y * istd) * gv4[k].y;
      xv4[k].z = (xv4[k].z * istd) * gv4[k].z;
      xv4[k].w = (xv4[k].w * istd) * gv4[k].w;
    }
  }
  // 3. amax of the token's row (every thread takes part: barriers follow)
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < F4; k++) {
    float t;
    t = dsl_abs(xv4[k].x); amax = t > amax ? t : amax;
    t = dsl_abs(xv4[k].y); amax = t > amax ? t : amax;
    t = dsl_abs(xv4[k].z); amax = t > amax ? t : amax;
    t = dsl_abs(xv4[k].w); amax = t > amax ? t : amax;
  }
  amax = nlg_block_max_f32<4, true>(amax, red2);
  const float g = nlg_gamma_of(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(amax))));
  const float ginv = 1.0f / g;
  if (!PLAIN && gamma_out && blockIdx.x == 0 && threadIdx.x == 0) gamma_out[tok] = g;
  // 4. quantise into LDS, one packed word per float4 (exact; see lane_est),
  //    stored already in the dots' operand order: a 16-column group's four
  //    words sit in the four lanes of a quad, and lane i keeps byte i of
  //    each (xpose4 across the quad, by DPP broadcasts)
  const bool fast = quant_fast(g);
  uint32_t *s_xq = (uint32_t *)s_xq4;
  const uint32_t qi = threadIdx.x & 3u;
  const uint32_t sel_lo = 0x0c0c0000u | ((4u + qi) << 8) | qi, sel_hi = 0x00000c0cu | ((4u + qi) << 24) | (qi << 16);
  uint32_t qw[F4];
  quant_words<F4>(xv4, g, ginv, fast, qw);
#pragma unroll
  for (int k = 0; k < F4; k++) {
    const uint32_t f = threadIdx.x + 256u * k;
    const uint32_t wd = qw[k];
    if (XPOSE_LOAD) {
      s_xq[f] = wd;
    } else {
      const uint32_t n0 = nlg_qperm<0x00>(wd), n1 = nlg_qperm<0x55>(wd);
      const uint32_t n2 = nlg_qperm<0xAA>(wd), n3 = nlg_qperm<0xFF>(wd);
      s_xq[f] = __builtin_amdgcn_perm(n1, n0, sel_lo) | __builtin_amdgcn_perm(n3, n2, sel_hi);
    }
  }
  __syncthreads();
  if (row0 >= a.out) return;  // wave-uniform, after the last barrier
  // 5. dots against the LDS activation, 6. reduce; lane r takes row r's
  //    exact accumulator
  int tl = 0;
  if (PACK) {
    int acc = 0;
#pragma unroll
    for (int k = 0; k < KPL; k++) {
      if ((uint32_t)(G * k) < nchunk) {  // wave-uniform: some lane's chunk is real
        const uint32_t c = pj + G * k, cc = c < nchunk ? c : nchunk - 1;
        const bool valid = c < nchunk;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint4 y = s_xq4[4 * cc + j];
          uint32_t w = j == 0 ? wv[k][0].x : j == 1 ? wv[k][0].y : j == 2 ? wv[k][0].z : wv[k][0].w;
          w = valid ? w : 0u;
          acc = wdot(w, y.x, y.y, y.z, y.w, acc);
        }
      }
    }
    // the row's G lanes: quads, then halves of 8 (mirror), then rows of 16
    acc += nlg_dpp<0xB1>(acc);                      // quad_perm [1,0,3,2]
    acc += nlg_dpp<0x4E>(acc);                      // quad_perm [2,3,0,1]
    if (G >= 8) acc += nlg_dpp<0x141>(acc);         // row_half_mirror
    if (G >= 16) acc += nlg_dpp<0x140>(acc);        // row_mirror
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int tot = __builtin_amdgcn_readlane(acc, r * G);
      tl = lane == r ? tot : tl;
    }
  } else {
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const uint32_t c = lane + 64 * i;
      if (c < nchunk) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint4 y = s_xq4[4 * c + j];
#pragma unroll
          for (int r = 0; r < R; r++) {
            const uint32_t w = j == 0 ? wv[r][i].x : j == 1 ? wv[r][i].y : j == 2 ? wv[r][i].z : wv[r][i].w;
            acc[r] = wdot(w, y.x, y.y, y.z, y.w, acc[r]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int tot = nlg_wave_sum_i32(acc[r]);
      tl = lane == r ? tot : tl;
    }
  }
  // Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc)   (kernels.el:633)
  const float val = __fadd_rn(bo, __fmul_rn(__fmul_rn(be, g), (float)(tl >> 6)));
  if (EPI == NLG_EPI_STORE || PLAIN || EPI == NLG_EPI_ARGMAX) {
    if (olive) y_out[(size_t)tok * ystride + orow] = val;
  }
  if (TIMED && lane == 0) {
    const unsigned long long t_end = __builtin_amdgcn_s_memrealtime();
    unsigned long long *ts = a.stamps + 2 * ((size_t)blockIdx.x * 4 + wvi);
    ts[0] = t_start;
    ts[1] = t_end;
  }
  if (EPI == NLG_EPI_RESID) {
    if (olive) y_out[(size_t)tok * ystride + orow] = __fadd_rn(rv, val);
  }
  if (EPI == NLG_EPI_SWIGLU || EPI == NLG_EPI_QKV) {
    // the other row of the pair (lane ^ 1)
    const float pv = __int_as_float(nlg_dpp<0xB1>(__float_as_int(val)));
    if (EPI == NLG_EPI_SWIGLU) {
      if (olive && !(lane & 1)) {
        const float sg = nlg_silu_gate(val);
        y_out[(size_t)tok * ystride + (orow >> 1)] = (val * sg) * pv;
      }
    } else if (olive) {
      // decode-rope: C[i0] = a0*cc - a1*ss; C[i1] = a0*ss + a1*cc
      const bool odd = lane & 1;
      const float a0 = odd ? pv : val, a1 = odd ? val : pv;
      const float rot = odd ? __fadd_rn(__fmul_rn(a0, ss), __fmul_rn(a1, cc))
                            : __fsub_rn(__fmul_rn(a0, cc), __fmul_rn(a1, ss));
      if (orow < a.nq) {
        y_out[(size_t)tok * ystride + orow] = rot;
      } else if (pos_ok) {
        const bool isk = orow < a.nq + a.nkv;
        const uint32_t sec = isk ? orow - a.nq : orow - a.nq - a.nkv;
        const uint32_t kh = sec / a.hd;
        const uint32_t sq = a.qper ? tok / a.qper : tok;
        const size_t at = (((size_t)sq * a.kvheads + kh) * a.max_seq + p) * a.hd + dd;
        if (isk) a.kc[at] = f32_to_f16_bits(rot);
        else a.vc[at] = f32_to_f16_bits(val);
      }
    }
  }
  if (EPI == NLG_EPI_ARGMAX) {
    // first maximum of the wave's rows (NaN never wins)
    float bv = -INFINITY;
    int32_t bi = -1;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val), r));
      if (row0 + r < a.out && (bi < 0 ? v == v : v > bv)) {
        bv = v;
        bi = (int32_t)(row0 + r);
      }
    }
    if (lane == 0) {
      a.pval[(size_t)tok * a.nparts + wave] = bv;
      a.pidx[(size_t)tok * a.nparts + wave] = bi;
    }
  }
}

// Each workgroup quantises the whole activation row, so fewer, fatter
// workgroups waste less -- down to about one workgroup per CU.  Measured
// at the decode shapes (graph-timed, weights streamed from HBM): 4 rows per
// wave for 2560..4096 outputs, 8 for the 13824-row gate|up and the LM head.
int nlg_fused_rows_per_wave(uint32_t out, int epi, uint32_t cols) {
  // the LM head: 16 rows per wave on rows of up to 3072 columns, the packed
  // form (128,256 x 2,560, one row, graph-timed with the argmax: 8 rows
  // 34.9 us, 16 30.6, 32 34.0; the quantisation as its own launch in front
  // of a prologue-free GEMV measured 32.0); wider rows keep 8, since 16 rows
  // of unpacked chunks there need 238+ VGPRs (two waves per SIMD or one).
  // cols 0 (unknown) answers 8: the most partials any call can leave.
  if (epi == NLG_EPI_ARGMAX) return out >= 32768 ? (cols && cols <= 3072 ? 16 : 8) : 4;
  if (epi == NLG_EPI_SWIGLU || epi == NLG_EPI_QKV) return out >= 8192 ? 8 : (out >= 2048 ? 4 : 2);
  return out >= 8192 ? 8 : (out >= 2048 ? 4 : (out >= 1024 ? 2 : 1));
}

// The row length picks the chunks per lane and the activation float4s per
// thread together (cols = 64 x chunks x CPL; cols <= 1024 x F4), so only the
// five pairs a row length can give are instantiated.
template <int PRO, int EPI, int R>
// The LDS row holds every word a thread quantises (256 F4 words, 1024 F4
// bytes): the words past the row are stored too (never read), so the
// stores need no per-thread condition.
static void fused_go(const FusedArgs &a, dim3 grid, hipStream_t st) {
  const dim3 blk(256);
  if (a.cols <= 2048) hipLaunchKernelGGL((k_tern_fused<R, 1, 2, PRO, EPI>), grid, blk, 2048, st, a);
  else if (a.cols <= 3072) hipLaunchKernelGGL((k_tern_fused<R, 1, 3, PRO, EPI>), grid, blk, 3072, st, a);
  else if (a.cols <= 4096) hipLaunchKernelGGL((k_tern_fused<R, 1, 4, PRO, EPI>), grid, blk, 4096, st, a);
  else if (a.cols <= 8192) hipLaunchKernelGGL((k_tern_fused<R, 2, 8, PRO, EPI>), grid, blk, 8192, st, a);
  else hipLaunchKernelGGL((k_tern_fused<R, 4, 16, PRO, EPI>), grid, blk, 16384, st, a);
}

uint32_t nlg_argmax_parts(uint32_t seq, uint32_t cols, uint32_t out) {
  if (nlg_batched(seq, cols)) return (out + 63) / 64;  // one per GEMM workgroup
  const uint32_t rpw = (uint32_t)nlg_fused_rows_per_wave(out, NLG_EPI_ARGMAX, cols);
  return (out + rpw - 1) / rpw;
}

int nlg_fused_launch(const FusedArgs &a0, int pro, int epi, int rpw, hipStream_t st) {
  FusedArgs a = a0;
  if (!a.seq || !a.out) return NLG_OK;
  if (nlg_batched(a.seq, a.cols)) return nlg_batched_launch(a, pro, epi, st);
  if (a.cols % 64 || a.cols > 16384 || !a.cols)
    return nlg_fail("fused ternary linear: cols must be a multiple of 64 in [64, 16384] (got %u)", a.cols);
  if (((uintptr_t)a.x & 15) || ((uintptr_t)a.w2 & 15) || (pro == NLG_PRO_RMS && ((uintptr_t)a.gain & 15)))
    return nlg_fail("fused ternary linear: x, w2 and gain must be 16-byte aligned");
  if (a.seq > 65535) return nlg_fail("fused ternary linear: seq %u > 65535", a.seq);
  a.wng = a.cols / 16;
  if (rpw <= 0) rpw = nlg_fused_rows_per_wave(a.out, epi, a.cols);
  if ((epi == NLG_EPI_SWIGLU || epi == NLG_EPI_QKV) && (rpw < 2 || a.out % 2))
    return nlg_fail("fused ternary linear: paired epilogues need an even row count");
  const dim3 grid(nlg_blocks(a.out, 4u * rpw), a.seq);
  // one (max, index) per wave that has rows
  if (epi == NLG_EPI_ARGMAX) a.nparts = (a.out + rpw - 1) / rpw;
#define PE(P, E)                                          \
  do {                                                    \
    switch (rpw) {                                        \
      case 1: fused_go<P, E, 1>(a, grid, st); break; \
      case 2: fused_go<P, E, 2>(a, grid, st); break; \
      case 8: fused_go<P, E, 8>(a, grid, st); break; \
      default: fused_go<P, E, 4>(a, grid, st); break; \
    }                                                     \
  } while (0)
  if (rpw != 1 && rpw != 2 && rpw != 4 && rpw != 8 && !(rpw == 16 && epi == NLG_EPI_ARGMAX))
    return nlg_fail("rows_per_wave must be 1, 2, 4 or 8 (or 16 for an argmax)");
  if (pro == NLG_PRO_NONE && epi == NLG_EPI_STORE && a.stamps && !a.bias && !a.beta_per_row && !a.gamma_out &&
      a.seq == 1)
    PE(NLG_PRO_NONE, NLG_EPI_STORE_TIMED);
  else if (pro == NLG_PRO_NONE && epi == NLG_EPI_STORE && !a.bias && !a.beta_per_row && !a.gamma_out)
    PE(NLG_PRO_NONE, NLG_EPI_STORE_PLAIN);
  else if (pro == NLG_PRO_NONE && epi == NLG_EPI_STORE) PE(NLG_PRO_NONE, NLG_EPI_STORE);
  else if (pro == NLG_PRO_RMS && epi == NLG_EPI_STORE) PE(NLG_PRO_RMS, NLG_EPI_STORE);
  else if (pro == NLG_PRO_NONE && epi == NLG_EPI_RESID) PE(NLG_PRO_NONE, NLG_EPI_RESID);
  else if (pro == NLG_PRO_RMS && epi == NLG_EPI_SWIGLU) PE(NLG_PRO_RMS, NLG_EPI_SWIGLU);
  else if (pro == NLG_PRO_NONE && epi == NLG_EPI_SWIGLU) PE(NLG_PRO_NONE, NLG_EPI_SWIGLU);
  else if (pro == NLG_PRO_RMS && epi == NLG_EPI_QKV) PE(NLG_PRO_RMS, NLG_EPI_QKV);
  else if (pro == NLG_PRO_RMS && epi == NLG_EPI_ARGMAX) {
    if (rpw == 16) fused_go<NLG_PRO_RMS, NLG_EPI_ARGMAX, 16>(a, grid, st);
    else PE(NLG_PRO_RMS, NLG_EPI_ARGMAX);
  }
  else if (pro == NLG_PRO_ATTN && epi == NLG_EPI_RESID) {
    if (!a.hd || a.hd % 4 || a.cols % a.hd || !a.attn_nc || a.attn_nc > NLG_ATTN_MAX_CHUNKS || !a.attn_mz)
      return nlg_fail("fused ternary linear: bad attention partials (hd %u, chunks %u)", a.hd, a.attn_nc);
    if (a.attn_nc == 3) PE(NLG_PRO_ATTN3, NLG_EPI_RESID);
    else PE(NLG_PRO_ATTN, NLG_EPI_RESID);
  }
  else return nlg_fail("fused ternary linear: unsupported prologue/epilogue %d/%d", pro, epi);
#undef PE
  NLG_LAUNCHED("fused ternary linear");
  return NLG_OK;
}

// ------------------------------------------------------ public entry points

extern "C" int nlg_rms_ternary_linear(const float *x, const float *gain, float eps, const uint32_t *w2,
                                      const float *bias, const float *beta, int beta_per_row, float *y,
                                      uint32_t seq, uint32_t out, uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  FusedArgs a{};
  a.x = x; a.gain = gain; a.eps = eps; a.w2 = w2; a.bias = bias; a.beta = beta;
  a.beta_per_row = beta_per_row; a.seq = seq; a.out = out; a.cols = cols;
  a.y = y; a.ystride = out;
  return nlg_fused_launch(a, NLG_PRO_RMS, NLG_EPI_STORE, 0, nlg_stream(stream));
}

extern "C" int nlg_ternary_linear_residual(const float *x, const uint32_t *w2, const float *bias,
                                           const float *beta, int beta_per_row, const float *res,
                                           float *y, uint32_t seq, uint32_t out, uint32_t cols,
                                           void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!res) return nlg_fail("ternary linear residual: res is null");
  FusedArgs a{};
  a.x = x; a.w2 = w2; a.bias = bias; a.beta = beta; a.beta_per_row = beta_per_row;
  a.seq = seq; a.out = out; a.cols = cols; a.y = y; a.ystride = out; a.res = res; a.rstride = out;
  return nlg_fused_launch(a, NLG_PRO_NONE, NLG_EPI_RESID, 0, nlg_stream(stream));
}

extern "C" int nlg_rms_ternary_swiglu(const float *x, const float *gain, float eps, const uint32_t *w2gu,
                                      const float *beta, int beta_per_row, float *h, uint32_t seq,
                                      uint32_t dff, uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  FusedArgs a{};
  a.x = x; a.gain = gain; a.eps = eps; a.w2 = w2gu; a.beta = beta; a.beta_per_row = beta_per_row;
  a.seq = seq; a.out = 2 * dff; a.cols = cols; a.y = h; a.ystride = dff;
  return nlg_fused_launch(a, gain ? NLG_PRO_RMS : NLG_PRO_NONE, NLG_EPI_SWIGLU, 0, nlg_stream(stream));
}

static int qkv_rope(const float *x, const float *gain, float eps, const uint32_t *w2qkv, const float *beta,
                    int beta_per_row, float *q, uint16_t *kcache, uint16_t *vcache, const float *rope_cos,
                    const float *rope_sin, const int32_t *pos, uint32_t rows, uint32_t qper, uint32_t heads,
                    uint32_t kvheads, uint32_t head_dim, uint32_t max_seq, uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!heads || !kvheads || !head_dim || head_dim % 2 || !max_seq)
    return nlg_fail("qkv: heads, kvheads, max_seq must be nonzero and head_dim even");
  if (qper && rows % qper) return nlg_fail("qkv: rows (%u) must be a multiple of qper (%u)", rows, qper);
  FusedArgs a{};
  a.x = x; a.gain = gain; a.eps = eps; a.w2 = w2qkv; a.beta = beta; a.beta_per_row = beta_per_row;
  a.seq = rows; a.nq = heads * head_dim; a.nkv = kvheads * head_dim; a.out = a.nq + 2 * a.nkv;
  a.cols = cols; a.y = q; a.ystride = a.nq; a.hd = head_dim; a.kvheads = kvheads; a.max_seq = max_seq;
  a.co = rope_cos; a.si = rope_sin; a.pos = pos; a.kc = kcache; a.vc = vcache; a.qper = qper;
  if (a.nq % 4 || a.nkv % 4) return nlg_fail("qkv: heads*head_dim and kvheads*head_dim must be multiples of 4");
  return nlg_fused_launch(a, NLG_PRO_RMS, NLG_EPI_QKV, 0, nlg_stream(stream));
}

extern "C" int nlg_rms_ternary_qkv_rope(const float *x, const float *gain, float eps, const uint32_t *w2qkv,
                                        const float *beta, int beta_per_row, float *q, uint16_t *kcache,
                                        uint16_t *vcache, const float *rope_cos, const float *rope_sin,
                                        const int32_t *pos, uint32_t seq, uint32_t heads,
                                        uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                                        uint32_t cols, void *stream) {
  return qkv_rope(x, gain, eps, w2qkv, beta, beta_per_row, q, kcache, vcache, rope_cos, rope_sin, pos, seq, 0,
                  heads, kvheads, head_dim, max_seq, cols, stream);
}

extern "C" int nlg_rms_ternary_qkv_rope_prompt(const float *x, const float *gain, float eps,
                                               const uint32_t *w2qkv, const float *beta, int beta_per_row,
                                               float *q, uint16_t *kcache, uint16_t *vcache,
                                               const float *rope_cos, const float *rope_sin, const int32_t *pos,
                                               uint32_t rows, uint32_t qper, uint32_t heads, uint32_t kvheads,
                                               uint32_t head_dim, uint32_t max_seq, uint32_t cols, void *stream) {
  if (!qper) return nlg_fail("qkv prompt: qper must be nonzero");
  return qkv_rope(x, gain, eps, w2qkv, beta, beta_per_row, q, kcache, vcache, rope_cos, rope_sin, pos, rows, qper,
                  heads, kvheads, head_dim, max_seq, cols, stream);
}

// ------------------------------------------------------------ sampling

// Greedy choice over the LM head's per-wave (max, index) pairs: the largest
// logit, the lowest index among equals; -1 marks a wave with no candidate.
__device__ __forceinline__ bool cand_better(float v, int32_t i, float bv, int32_t bi) {
  if (i < 0) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

__device__ void block_argmax(float &v, int32_t &i, float *sv, int32_t *si) {
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int32_t oi = __shfl_xor(i, off);
    if (cand_better(ov, oi, v, i)) { v = ov; i = oi; }
  }
  const int nw = blockDim.x >> 6, w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = i; }
  __syncthreads();
  v = sv[0]; i = si[0];
  for (int k = 1; k < nw; k++)
    if (cand_better(sv[k], si[k], v, i)) { v = sv[k]; i = si[k]; }
}

__global__ __launch_bounds__(1024) void k_argmax_parts(const float *pval, const int32_t *pidx,
                                                       uint32_t nparts, int32_t *out) {
  __shared__ float sv[16];
  __shared__ int32_t si[16];
  const uint32_t t = blockIdx.x;
  float v = -INFINITY;
  int32_t i = -1;
  for (uint32_t j = threadIdx.x; j < nparts; j += blockDim.x) {
    const float ov = pval[(size_t)t * nparts + j];
    const int32_t oi = pidx[(size_t)t * nparts + j];
    if (cand_better(ov, oi, v, i)) { v = ov; i = oi; }
  }
  block_argmax(v, i, sv, si);
  if (threadIdx.x == 0) out[t] = i;
}

extern "C" size_t nlg_rms_ternary_argmax_workspace(uint32_t seq, uint32_t vocab) {
  // the larger of the two forms' partial counts, whatever cols the call uses
  const int rpw = nlg_fused_rows_per_wave(vocab, NLG_EPI_ARGMAX, 0);
  size_t nparts = (vocab + rpw - 1) / rpw;
  if ((size_t)(vocab + 63) / 64 > nparts) nparts = (vocab + 63) / 64;
  return (size_t)seq * nparts * 8;
}

extern "C" int nlg_rms_ternary_argmax(const float *x, const float *gain, float eps, const uint32_t *w2,
                                      const float *beta, int beta_per_row, float *logits,
                                      int32_t *argmax, uint32_t seq, uint32_t vocab, uint32_t cols,
                                      void *workspace, size_t workspace_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!seq || !vocab) return NLG_OK;
  const size_t need = nlg_rms_ternary_argmax_workspace(seq, vocab);
  if (!workspace || workspace_bytes < need)
    return nlg_fail("rms ternary argmax: needs a %zu-byte workspace", need);
  hipStream_t st = nlg_stream(stream);
  const int rpw = nlg_fused_rows_per_wave(vocab, NLG_EPI_ARGMAX, cols);
  const uint32_t nparts = nlg_argmax_parts(seq, cols, vocab);
  FusedArgs a{};
  a.x = x; a.gain = gain; a.eps = eps; a.w2 = w2; a.beta = beta; a.beta_per_row = beta_per_row;
  a.seq = seq; a.out = vocab; a.cols = cols; a.y = logits; a.ystride = vocab;
  a.pval = (float *)workspace;
  a.pidx = (int32_t *)((char *)workspace + (size_t)seq * nparts * 4);
  if (nlg_fused_launch(a, NLG_PRO_RMS, NLG_EPI_ARGMAX, rpw, st)) return NLG_ERR;
  hipLaunchKernelGGL(k_argmax_parts, dim3(seq), dim3(1024), 0, st, a.pval, a.pidx, nparts, argmax);
  NLG_LAUNCHED("argmax");
  return NLG_OK;
}

