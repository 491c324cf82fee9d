// nlg_gemm.hip -- f32 GEMM behind matmul, matmul-tiled, matmul-reg, linear
// (lisp/nelisp-gpu-kernels.el:17-27, :71-107, :129).
//
// The reference has three schedules of the same product (naive, 16x16 LDS
// tiles, 4x4 register tiles) plus `linear` (X.W^T + bias).  One 64x64-tile
// kernel serves all four: 256 threads, each accumulating a 4x4 block strided
// by 16 so LDS reads are conflict-free, 16-deep K steps staged through LDS.
// Accumulation uses FMA; parity with the serial reference is by tolerance,
// and integer-valued inputs (host/vkmatmul.c:92-93) are exact.
#include "nlg_internal.h"

template <bool TRANS_B, bool BIAS>
__global__ __launch_bounds__(256) void k_sgemm(const float *__restrict__ A, const float *__restrict__ B,
                                               const float *__restrict__ bias, float *__restrict__ C,
                                               uint32_t M, uint32_t N, uint32_t K) {
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const uint32_t m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const uint32_t t = threadIdx.x, tx = t % 16, ty = t / 16;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;

  for (uint32_t k0 = 0; k0 < K; k0 += 16) {
    {  // A tile: 64 rows x 16 k; thread t loads row t/4, k (t%4)*4 .. +3
      const uint32_t m = t / 4, kq = (t % 4) * 4;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t gm = m0 + m, gk = k0 + kq + q;
        As[kq + q][m] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.0f;
      }
    }
    if (TRANS_B) {  // W is N x K (linear): thread t loads n t/4, k (t%4)*4 .. +3
      const uint32_t n = t / 4, kq = (t % 4) * 4;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t gn = n0 + n, gk = k0 + kq + q;
        Bs[kq + q][n] = (gn < N && gk < K) ? B[(size_t)gn * K + gk] : 0.0f;
      }
    } else {  // B is K x N: thread t loads k t/16, n (t%16)*4 .. +3
      const uint32_t kk = t / 16, nq = (t % 16) * 4;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t gk = k0 + kk, gn = n0 + nq + q;
        Bs[kk][nq + q] = (gk < K && gn < N) ? B[(size_t)gk * N + gn] : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t gm = m0 + ty + 16 * i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t gn = n0 + tx + 16 * j;
      if (gn < N) C[(size_t)gm * N + gn] = BIAS ? __fadd_rn(bias[gn], acc[i][j]) : acc[i][j];
    }
  }
}

static int sgemm(const float *A, const float *B, const float *bias, float *C, uint32_t M, uint32_t N,
                 uint32_t K, bool trans_b, hipStream_t st, const char *name) {
  if (!M || !N) return NLG_OK;
  dim3 g(nlg_blocks(N, 64), nlg_blocks(M, 64)), b(256);
  if (trans_b) {
    if (bias) hipLaunchKernelGGL((k_sgemm<true, true>), g, b, 0, st, A, B, bias, C, M, N, K);
    else hipLaunchKernelGGL((k_sgemm<true, false>), g, b, 0, st, A, B, bias, C, M, N, K);
  } else {
    hipLaunchKernelGGL((k_sgemm<false, false>), g, b, 0, st, A, B, bias, C, M, N, K);
  }
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

// matmul (kernels.el:17-27): A B C; push (M K N); one invocation per C element
int L_matmul(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], K = p[1], N = p[2];
  if (nlg_domain((uint64_t)M * N, groups) < (uint64_t)M * N)
    return nlg_fail("matmul: %u groups do not cover %u x %u outputs", groups, M, N);
  if (mm_check(b, M, K, N, "matmul")) return NLG_ERR;
  return sgemm((const float *)b[0].ptr, (const float *)b[1].ptr, nullptr, (float *)b[2].ptr, M, N, K,
               false, st, "matmul");
}
// matmul-tiled (kernels.el:82-107): one 16x16 workgroup per C tile
int L_matmul_tiled(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], K = p[1], N = p[2];
  const uint64_t tiles = (uint64_t)((M + 15) / 16) * ((N + 15) / 16);
  if (groups < tiles) return nlg_fail("matmul-tiled: %u groups do not cover %llu tiles", groups,
                                      (unsigned long long)tiles);
  if (mm_check(b, M, K, N, "matmul-tiled")) return NLG_ERR;
  return sgemm((const float *)b[0].ptr, (const float *)b[1].ptr, nullptr, (float *)b[2].ptr, M, N, K,
               false, st, "matmul-tiled");
}
// matmul-reg (kernels.el:129): a 4x4 micro-tile per invocation; the
// reference writes past row ends unless M and N are multiples of 4.
int L_matmul_reg(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], K = p[1], N = p[2];
  if (M % 4 || N % 4) return nlg_fail("matmul-reg: M and N must be multiples of 4 (got %u, %u)", M, N);
  const uint64_t blocks = (uint64_t)(M / 4) * (N / 4);
  if (nlg_domain(blocks, groups) < blocks) return nlg_fail("matmul-reg: groups do not cover the output");
  if (mm_check(b, M, K, N, "matmul-reg")) return NLG_ERR;
  return sgemm((const float *)b[0].ptr, (const float *)b[1].ptr, nullptr, (float *)b[2].ptr, M, N, K,
               false, st, "matmul-reg");
}
// linear (kernels.el:71-81): X W B C; push (M IN OUT); C = X.W^T + B
int L_linear(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], IN = p[1], OUT = p[2];
  if (nlg_domain((uint64_t)M * OUT, groups) < (uint64_t)M * OUT)
    return nlg_fail("linear: groups do not cover the output");
  const char *k = "linear";
  if (nlg_need(b, 0, (uint64_t)M * IN, k) || nlg_need(b, 1, (uint64_t)OUT * IN, k) ||
      nlg_need(b, 2, OUT, k) || nlg_need(b, 3, (uint64_t)M * OUT, k))
    return NLG_ERR;
  return sgemm((const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr,
               (float *)b[3].ptr, M, OUT, IN, true, st, k);
}
