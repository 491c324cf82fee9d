// nlg_gemm.hip -- f32 GEMM behind matmul, matmul-tiled, matmul-reg, linear
// (lisp/nelisp-gpu-kernels.el:17-27, :71-107, :129).
//
// Each output element is one dependent chain of f32 additions in the
// reference, so one kernel serves all four names with the reference's own
// summation order per name (bit-identical results):
//   matmul, matmul-reg, linear  acc = acc + a*b for k = 0..K-1 (acc starts at
//                               0, or at the bias for linear);
//   matmul-tiled                per 16-wide k tile, p0 + (p1 + (... + (p14 +
//                               p15))) added to acc (the tile sum the
//                               reference writes out, zero products past K).
// The chain length bounds the time, not the flops, so the work is spread
// as wide as it goes: one 256-thread workgroup per 16 x 16 output tile (a
// 256^3 product is 256 workgroups, one per CU), one output per thread, the
// tile's A rows and B columns for 256 values of k staged through LDS with
// every global load of a chunk issued before the first is used.
//
// Partial grids: a dispatch of `groups` workgroups covers only the outputs
// the reference's invocations gid < 64*groups (matmul-tiled: workgroups
// wg < groups) would write; the rest of C is left as it was.
#include "nlg_internal.h"

#define MM_T 16    // output tile edge
#define MM_KC 256  // k per LDS stage

enum { MM_SERIAL = 0, MM_TILE16 = 1 };
// which outputs a partial grid covers: by row-major index, by 4x4 block
// index (matmul-reg), or by 16x16 tile index (matmul-tiled)
enum { LIM_INDEX = 0, LIM_BLOCK4 = 1, LIM_TILE16 = 2 };

template <int ORDER, bool TRANS_B, bool BIAS>
__global__ __launch_bounds__(256) void k_mm(const float *__restrict__ A, const float *__restrict__ B,
                                            const float *__restrict__ bias, float *__restrict__ C, uint32_t M,
                                            uint32_t N, uint32_t K, int lim_mode, uint64_t lim) {
  __shared__ float As[MM_T][MM_KC + 1];
  __shared__ float Bs[MM_KC][MM_T + 1];
  const uint32_t t = threadIdx.x, tx = t & 15, ty = t >> 4;
  const uint32_t m0 = blockIdx.y * MM_T, n0 = blockIdx.x * MM_T;
  const uint32_t row = m0 + ty, col = n0 + tx;
  float acc = 0.0f;
  if (BIAS) acc = col < N ? bias[col] : 0.0f;
  for (uint32_t k0 = 0; k0 < K; k0 += MM_KC) {
    const uint32_t kc = K - k0 < MM_KC ? K - k0 : MM_KC;
    float ra[MM_T], rb[MM_T];
    // A rows m0..m0+15, k0..k0+255: lane t reads column k0+t of each row
#pragma unroll
    for (int j = 0; j < MM_T; j++) {
      const uint32_t r = m0 + j;
      ra[j] = (r < M && t < kc) ? A[(size_t)r * K + k0 + t] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < MM_T; j++) {
      if (TRANS_B) {  // W [N x K]: lane t reads k0+t of rows n0..n0+15
        const uint32_t c = n0 + j;
        rb[j] = (c < N && t < kc) ? B[(size_t)c * K + k0 + t] : 0.0f;
      } else {  // B [K x N]: lanes read 16 consecutive columns of 16 k rows
        const uint32_t kk = 16 * j + (t >> 4), c = n0 + (t & 15);
        rb[j] = (kk < kc && c < N) ? B[(size_t)(k0 + kk) * N + c] : 0.0f;
      }
    }
    __syncthreads();  // the previous stage has been consumed
#pragma unroll
    for (int j = 0; j < MM_T; j++) {
      As[j][t] = ra[j];
      if (TRANS_B) Bs[t][j] = rb[j];
      else Bs[16 * j + (t >> 4)][t & 15] = rb[j];
    }
    __syncthreads();
    if (ORDER == MM_SERIAL) {
      // acc = acc + a*b, k ascending (kernels.el:24-26, :78-80); unrolled so
      // the LDS reads run well ahead of the dependent adds
#pragma unroll 32
      for (uint32_t k = 0; k < kc; k++) acc = __fadd_rn(acc, __fmul_rn(As[ty][k], Bs[k][tx]));
    } else {
      // kernels.el:99-104: acc + (p0 + (p1 + ... (p14 + p15))) per tile of 16
      for (uint32_t kb = 0; kb < kc; kb += 16) {
        float s = __fmul_rn(As[ty][kb + 15], Bs[kb + 15][tx]);
#pragma unroll
        for (int q = 14; q >= 0; q--) s = __fadd_rn(__fmul_rn(As[ty][kb + q], Bs[kb + q][tx]), s);
        acc = __fadd_rn(acc, s);
      }
    }
  }
  if (row >= M || col >= N) return;
  uint64_t at;
  if (lim_mode == LIM_INDEX) at = (uint64_t)row * N + col;
  else if (lim_mode == LIM_BLOCK4) at = (uint64_t)(row / 4) * ((N + 3) / 4) + col / 4;
  else at = (uint64_t)(row / 16) * ((N + 15) / 16) + col / 16;
  if (at < lim) C[(size_t)row * N + col] = acc;
}

template <int ORDER>
static void mm_go(const float *A, const float *B, const float *bias, float *C, uint32_t M, uint32_t N, uint32_t K,
                  bool trans_b, int lim_mode, uint64_t lim, hipStream_t st) {
  const dim3 g(nlg_blocks(N, MM_T), nlg_blocks(M, MM_T)), b(256);
  if (trans_b) {
    if (bias) hipLaunchKernelGGL((k_mm<ORDER, true, true>), g, b, 0, st, A, B, bias, C, M, N, K, lim_mode, lim);
    else hipLaunchKernelGGL((k_mm<ORDER, true, false>), g, b, 0, st, A, B, bias, C, M, N, K, lim_mode, lim);
  } else {
    hipLaunchKernelGGL((k_mm<ORDER, false, false>), g, b, 0, st, A, B, bias, C, M, N, K, lim_mode, lim);
  }
}

static int mm(const float *A, const float *B, const float *bias, float *C, uint32_t M, uint32_t N, uint32_t K,
              bool trans_b, int order, int lim_mode, uint64_t lim, hipStream_t st, const char *name) {
  if (!M || !N || !lim) return NLG_OK;
  if (nlg_blocks(M, MM_T) > 65535) return nlg_fail("%s: M = %u is too large", name, M);
  if (order == MM_TILE16) mm_go<MM_TILE16>(A, B, bias, C, M, N, K, trans_b, lim_mode, lim, st);
  else mm_go<MM_SERIAL>(A, B, bias, C, M, N, K, trans_b, lim_mode, lim, st);
  NLG_LAUNCHED(name);
  return NLG_OK;
}

static int mm_check(const nlg_buffer *b, uint32_t M, uint32_t K, uint32_t N, const char *k) {
  if (nlg_need(b, 0, (uint64_t)M * K, k) || nlg_need(b, 1, (uint64_t)K * N, k) ||
      nlg_need(b, 2, (uint64_t)M * N, k))
    return NLG_ERR;
  if ((uint64_t)M * N > 0xffffffffull) return nlg_fail("%s: M*N exceeds 2^32", k);
  return NLG_OK;
}

// matmul (kernels.el:17-27): A B C; push (M K N); invocation idx < M*N
// writes C[idx]
int L_matmul(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], K = p[1], N = p[2];
  if (mm_check(b, M, K, N, "matmul")) return NLG_ERR;
  return mm((const float *)b[0].ptr, (const float *)b[1].ptr, nullptr, (float *)b[2].ptr, M, N, K, false,
            MM_SERIAL, LIM_INDEX, nlg_domain((uint64_t)M * N, groups), st, "matmul");
}
// matmul-tiled (kernels.el:82-107): workgroup wg (of groups) writes C tile wg
int L_matmul_tiled(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], K = p[1], N = p[2];
  if (mm_check(b, M, K, N, "matmul-tiled")) return NLG_ERR;
  return mm((const float *)b[0].ptr, (const float *)b[1].ptr, nullptr, (float *)b[2].ptr, M, N, K, false,
            MM_TILE16, LIM_TILE16, groups, st, "matmul-tiled");
}
// matmul-reg (kernels.el:129): invocation idx writes the 4x4 block idx (row
// block idx / ceil(N/4)); the reference writes past row ends unless M and N
// are multiples of 4, so other shapes are refused.
int L_matmul_reg(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], K = p[1], N = p[2];
  if (M % 4 || N % 4) return nlg_fail("matmul-reg: M and N must be multiples of 4 (got %u, %u)", M, N);
  if (mm_check(b, M, K, N, "matmul-reg")) return NLG_ERR;
  const uint64_t blocks = (uint64_t)(M / 4) * (N / 4);
  return mm((const float *)b[0].ptr, (const float *)b[1].ptr, nullptr, (float *)b[2].ptr, M, N, K, false,
            MM_SERIAL, LIM_BLOCK4, nlg_domain(blocks, groups), st, "matmul-reg");
}
// linear (kernels.el:71-81): X W B C; push (M IN OUT); C = B + X.W^T,
// invocation idx < M*OUT writes C[idx]
int L_linear(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], IN = p[1], OUT = p[2];
  const char *k = "linear";
  if (nlg_need(b, 0, (uint64_t)M * IN, k) || nlg_need(b, 1, (uint64_t)OUT * IN, k) ||
      nlg_need(b, 2, OUT, k) || nlg_need(b, 3, (uint64_t)M * OUT, k))
    return NLG_ERR;
  if ((uint64_t)M * OUT > 0xffffffffull) return nlg_fail("linear: M*OUT exceeds 2^32");
  return mm((const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr, (float *)b[3].ptr, M,
            OUT, IN, true, MM_SERIAL, LIM_INDEX, nlg_domain((uint64_t)M * OUT, groups), st, k);
}
