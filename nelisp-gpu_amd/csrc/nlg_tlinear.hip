// nlg_tlinear.hip -- the transposed (input-gradient) linears, by name:
//
//   ternary-rows-t (kernels.el:748-775)  X[p,i] = sum_o w(o,i) * (BETA[o*nblk + i/128] * G[p,o])
//   dp4a-rows-t    (kernels.el:777-810)  X[p,i] = sum_o w(o,i) * (BETA[o] * G[p,o])
//
// One invocation per output element, as the reference: each column's sum
// runs over the rows o in order with one rounding per product and per add,
// so the result is bit-identical.  A wave's 64 columns share 4 (2-bit) or 16
// (int8-lane) weight words per row, read as broadcasts.  BETA * G is rounded
// once per row, as the reference's nesting rounds it.
#include "nlg_internal.h"

namespace {

struct TArgs {
  const uint32_t *wp;
  const float *beta, *g;
  float *x;
  uint32_t nwp, nbeta, ng_, nx;  // buffer lengths (floats)
  uint32_t out, cols, nblk, seq;
  uint32_t stride;  // weight row stride in words (the push's wng / ng)
  uint32_t wcols;   // words a position's columns occupy: ceil(cols / FPW)
  uint32_t domain;  // X elements written: min(seq*cols, 64*groups)
};

__device__ __forceinline__ float tld(const float *p, uint32_t n, uint32_t i) { return i < n ? p[i] : 0.0f; }
__device__ __forceinline__ uint32_t tldu(const uint32_t *p, uint32_t n, uint32_t i) { return i < n ? p[i] : 0u; }

// FPW: columns per word (16 for 2-bit fields, 4 for int8 lanes).  One lane
// per output element, as the reference; the rows go in groups of 32 whose
// loads are all issued before the group's adds, so the in-order sum is not
// one memory round trip per row.
template <int FPW>
__global__ __launch_bounds__(256) void k_rows_t(TArgs a) {
  const uint64_t lid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (lid >= (uint64_t)a.seq * a.cols) return;
  const uint32_t p = (uint32_t)(lid / a.cols), i = (uint32_t)(lid % a.cols);
  const uint32_t wi = i / FPW, f = i % FPW;
  const uint32_t blk = FPW == 16 ? i / 128 : 0u;  // the column's scale block (ternary-rows-t)
  const uint32_t gb = p * a.out;
  float acc = 0.0f;
  constexpr int U = 32;
  for (uint32_t o0 = 0; o0 < a.out; o0 += U) {
    uint32_t wv[U];
    float bv[U], gv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t o = o0 + u;  // rows past `out` are loaded (bounds-checked) but not added
      wv[u] = tldu(a.wp, a.nwp, o * a.stride + wi);
      bv[u] = tld(a.beta, a.nbeta, FPW == 16 ? o * a.nblk + blk : o);
      gv[u] = tld(a.g, a.ng_, gb + o);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      float sv;
      if (FPW == 16) sv = (float)((int32_t)(wv[u] << (30 - 2 * f)) >> 30);  // the field, sign-extended
      else sv = (float)(int32_t)(int8_t)(uint8_t)(wv[u] >> (8 * f));        // (b + 128) % 256 - 128
      const float t = __fmul_rn(sv, __fmul_rn(bv[u], gv[u]));
      if (o0 + u < a.out) acc = __fadd_rn(acc, t);
    }
  }
  const uint32_t idx = p * a.cols + i;
  if (idx < a.domain && idx < a.nx) a.x[idx] = acc;
}

int rows_t(const nlg_buffer *b, uint32_t out, uint32_t cols, uint32_t nblk, uint32_t stride, uint32_t seq,
           uint32_t groups, hipStream_t st, bool two_bit, const char *k) {
  TArgs a;
  a.wp = (const uint32_t *)b[0].ptr; a.nwp = b[0].nfloats;
  a.beta = (const float *)b[1].ptr; a.nbeta = b[1].nfloats;
  a.g = (const float *)b[2].ptr; a.ng_ = b[2].nfloats;
  a.x = (float *)b[3].ptr; a.nx = b[3].nfloats;
  a.out = out; a.cols = cols; a.nblk = nblk; a.seq = seq; a.stride = stride;
  const uint64_t dom = nlg_domain((uint64_t)seq * cols, groups);
  if (!dom || !cols) return NLG_OK;
  a.domain = (uint32_t)dom;
  a.wcols = two_bit ? (cols + 15) / 16 : (cols + 3) / 4;
  const uint32_t seqs = (uint32_t)((dom + cols - 1) / cols);
  a.seq = seqs < seq ? seqs : seq;  // positions with an element in the domain
  const uint64_t nw = (uint64_t)a.seq * cols;
  const dim3 grid((unsigned)((nw + 255) / 256)), blk(256);
  if (two_bit) hipLaunchKernelGGL(k_rows_t<16>, grid, blk, 0, st, a);
  else hipLaunchKernelGGL(k_rows_t<4>, grid, blk, 0, st, a);
  NLG_LAUNCHED(k);
  return NLG_OK;
}

}  // namespace

// ternary-rows-t: WP BETA G X; push (out cols nblk wng seq)
int L_ternary_rows_t(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return rows_t(b, p[0], p[1], p[2], p[3], p[4], groups, st, true, "ternary-rows-t");
}
// dp4a-rows-t: WP BETA G X; push (out cols ng seq)
int L_dp4a_rows_t(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return rows_t(b, p[0], p[1], 0, p[2], p[3], groups, st, false, "dp4a-rows-t");
}
