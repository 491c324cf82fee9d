// nlg_tlinear.hip -- the transposed (input-gradient) linears, by name:
//
//   ternary-rows-t (kernels.el:748-775)  X[p,i] = sum_o w(o,i) * (BETA[o*nblk + i/128] * G[p,o])
//   dp4a-rows-t    (kernels.el:777-810)  X[p,i] = sum_o w(o,i) * (BETA[o] * G[p,o])
//
// Each column's sum runs over the rows o in order with one rounding per
// product and per add, as the reference's invocation does, so the result is
// bit-identical.  BETA * G is rounded once per row, as the reference's
// nesting rounds it.
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

// FPW: columns per word (16 for 2-bit fields, 4 for int8 lanes).  Each
// column's sum is one chain of `out` dependent adds, so the kernel is built
// around that chain: a workgroup owns CG columns of one position; it first
// stages the weight words of its columns and the products BETA*G of up to RS
// rows in LDS (every load issued up front: one memory round trip), then
// three producer waves turn a CH-row chunk into the products
// t = field * (BETA*G) while the consumer wave adds the previous chunk's,
// row after row, one LDS read per four rows.  Same roundings in the same
// order as the reference, so the result is bit-identical.
constexpr int RT_RS = 2560;       // rows staged per pass (a multiple of 256)
constexpr int RT_CH = 192;        // rows per product chunk (a multiple of 32)
constexpr int RT_TP = RT_CH + 4;  // padded pitch of a column's products

template <int FPW>
__global__ __launch_bounds__(256) void k_rows_t(TArgs a) {
  constexpr int CG = FPW == 16 ? 64 : 32;  // columns per workgroup
  constexpr int NWD = CG / FPW;            // weight words per row and workgroup (4 or 8)
  constexpr int LR = RT_RS / 256;          // staged rows per thread
  constexpr int NT = (RT_CH / 4 * NWD + 191) / 192;  // producer tasks (4 rows x 1 word) per thread
  // 16-byte aligned: rows are read and written four at a time
  __shared__ __align__(16) uint32_t s_w[NWD * RT_RS];  // word-major: s_w[wd * RS + row]
  __shared__ __align__(16) float s_bg[RT_RS];
  __shared__ __align__(16) float s_t[2][CG * RT_TP];  // column-major products: s_t[b][col * TP + row]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t c0 = blockIdx.x * CG, p = blockIdx.y;
  const uint32_t wi0 = c0 / FPW;
  const uint32_t blk = FPW == 16 ? c0 / 128 : 0u;  // CG columns lie in one 128-column block
  const uint32_t gb = p * a.out;
  // rows' words as 16-byte loads when every row's piece is 16-byte aligned and inside the buffer
  const bool vec = ((uintptr_t)a.wp & 15) == 0 && a.stride % 4 == 0 &&
                   (uint64_t)(a.out - 1) * a.stride + wi0 + NWD <= a.nwp;
  float acc = 0.0f;  // the consumer lane's column
  for (uint32_t r0 = 0; r0 < a.out; r0 += RT_RS) {
    const uint32_t nr = a.out - r0 < (uint32_t)RT_RS ? a.out - r0 : (uint32_t)RT_RS;
    if (r0) __syncthreads();  // the previous pass's readers are done with s_w / s_bg
    // 1. stage rows tid + 256 k: all loads first (in bounds), then the LDS stores
    uint32_t wv[LR][NWD];
    float bv[LR], gv[LR];
    if (vec) {
#pragma unroll
      for (int k = 0; k < LR; k++) {
        const uint32_t rr = threadIdx.x + 256u * k, o = r0 + (rr < nr ? rr : nr - 1);
        const uint4 *src = (const uint4 *)(a.wp + (size_t)o * a.stride + wi0);
#pragma unroll
        for (int q = 0; q < NWD / 4; q++) {
          const uint4 v = src[q];
          wv[k][4 * q] = v.x; wv[k][4 * q + 1] = v.y; wv[k][4 * q + 2] = v.z; wv[k][4 * q + 3] = v.w;
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < LR; k++) {
        const uint32_t rr = threadIdx.x + 256u * k, o = r0 + (rr < nr ? rr : nr - 1);
#pragma unroll
        for (int j = 0; j < NWD; j++) wv[k][j] = tldu(a.wp, a.nwp, o * a.stride + wi0 + j);
      }
    }
#pragma unroll
    for (int k = 0; k < LR; k++) {
      const uint32_t rr = threadIdx.x + 256u * k, o = r0 + (rr < nr ? rr : nr - 1);
      bv[k] = tld(a.beta, a.nbeta, FPW == 16 ? o * a.nblk + blk : o);
      gv[k] = tld(a.g, a.ng_, gb + o);
    }
#pragma unroll
    for (int k = 0; k < LR; k++) {
#pragma unroll
      for (int j = 0; j < NWD; j++) s_w[j * RT_RS + threadIdx.x + 256u * k] = wv[k][j];
      s_bg[threadIdx.x + 256u * k] = __fmul_rn(bv[k], gv[k]);
    }
    __syncthreads();
    // 2. chunks: producers (waves 1..3) fill chunk c+1 while the consumer adds chunk c
    const uint32_t nch = (nr + RT_CH - 1) / RT_CH;
    auto produce = [&](uint32_t ch) {
      float *dst = s_t[ch & 1];
      // task (row quad, word): consecutive threads take consecutive quads
      uint4 wq[NT];
      float4 bq[NT];
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const uint32_t k = threadIdx.x - 64 + 192u * j;
        const uint32_t kc = k < (uint32_t)(RT_CH / 4 * NWD) ? k : 0u;
        const uint32_t q = kc % (RT_CH / 4), wd = kc / (RT_CH / 4);
        // rows past the pass (row >= nr, or even >= RS in the last chunk) give
        // products the consumer never adds; their reads stay inside the arrays
        const uint32_t row = ch * RT_CH + 4 * q;
        const uint32_t rc = row < (uint32_t)RT_RS ? row : (uint32_t)RT_RS - 4;
        wq[j] = *(const uint4 *)(s_w + wd * RT_RS + rc);
        bq[j] = *(const float4 *)(s_bg + rc);
      }
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const uint32_t k = threadIdx.x - 64 + 192u * j;
        if (k < (uint32_t)(RT_CH / 4 * NWD)) {
          const uint32_t q = k % (RT_CH / 4), wd = k / (RT_CH / 4);
          const uint32_t ws[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
          const float bs[4] = {bq[j].x, bq[j].y, bq[j].z, bq[j].w};
#pragma unroll
          for (int f = 0; f < FPW; f++) {
            float tv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
              float sv;
              if (FPW == 16) sv = (float)((int32_t)(ws[e] << (30 - 2 * f)) >> 30);  // the field, sign-extended
              else sv = (float)(int32_t)(int8_t)(uint8_t)(ws[e] >> (8 * f));        // (b + 128) % 256 - 128
              tv[e] = __fmul_rn(sv, bs[e]);
            }
            *(float4 *)(dst + (wd * FPW + f) * RT_TP + 4 * q) = make_float4(tv[0], tv[1], tv[2], tv[3]);
          }
        }
      }
    };
    if (w > 0) produce(0);
    __syncthreads();
    for (uint32_t ch = 0; ch < nch; ch++) {
      if (w == 0) {
        if (lane < CG) {
          const float *src = s_t[ch & 1] + lane * RT_TP;
          const uint32_t cnt = nr - ch * RT_CH < (uint32_t)RT_CH ? nr - ch * RT_CH : (uint32_t)RT_CH;
          if (cnt == (uint32_t)RT_CH) {
            // the next 32 rows' reads are in flight while these 32 are added
            constexpr int GR = 8;  // float4 reads per group
            float4 cur[GR], nxt[GR];
#pragma unroll
            for (int j = 0; j < GR; j++) cur[j] = *(const float4 *)(src + 4 * j);
#pragma unroll
            for (int g = 0; g < RT_CH / (4 * GR); g++) {
              if (g + 1 < RT_CH / (4 * GR)) {
#pragma unroll
                for (int j = 0; j < GR; j++) nxt[j] = *(const float4 *)(src + 4 * (GR * (g + 1) + j));
              }
              __builtin_amdgcn_sched_barrier(0);  // keep this order: reads, then the adds
#pragma unroll
              for (int j = 0; j < GR; j++) {
                acc = __fadd_rn(acc, cur[j].x);
                acc = __fadd_rn(acc, cur[j].y);
                acc = __fadd_rn(acc, cur[j].z);
                acc = __fadd_rn(acc, cur[j].w);
              }
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int j = 0; j < GR; j++) cur[j] = nxt[j];
            }
          } else {
            for (uint32_t r = 0; r < cnt; r++) acc = __fadd_rn(acc, src[r]);  // only the rows that exist
          }
        }
      } else if (ch + 1 < nch) {
        produce(ch + 1);
      }
      __syncthreads();
    }
  }
  if (w == 0 && lane < CG) {
    const uint32_t i = c0 + lane, idx = p * a.cols + i;
    if (i < a.cols && idx < a.domain && idx < a.nx) a.x[idx] = acc;
  }
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
  const uint32_t cg = two_bit ? 64u : 32u;
  const dim3 grid((cols + cg - 1) / cg, a.seq), blk(256);
  if (a.seq > 65535) return nlg_fail("%s: %u positions > 65535", k, a.seq);
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
