// nlg_rows.hip -- row reductions: softmax, RMSNorm (istd, per-head).
//
// The reference gives each row to one invocation, which walks it serially
// three times (softmax, kernels.el:28-42).  Here a workgroup owns a row: the
// row is read from HBM once into registers (16 floats per thread at 4096
// columns, non-temporal float4 loads), reduced with DPP within waves and LDS
// across them, and written once (non-temporal stores) -- 8 bytes of traffic
// per element, the minimum for an in-place softmax.  Reduction order differs from the serial reference, so
// parity is by tolerance (<= 1e-5 relative for softmax, 1e-4 for RMSNorm).
#include <math.h>

#include "nlg_internal.h"

#define EPS6 0.000001f

// The reference's max starts from the first element and only moves on a
// strict `>`: NaNs are never selected, except that a NaN first element stays.
template <int EPT, bool V4>
__global__ __launch_bounds__(256) void k_softmax_reg(const float *a, float *c, uint32_t rows,
                                                     uint32_t n) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const float *ar = a + (size_t)row * n;
  float *cr = c + (size_t)row * n;
  const float first = ar[0];
  float v[EPT];
  float mx = -INFINITY;
  if (V4) {
#pragma unroll
    for (int k = 0; k < EPT / 4; k++) {
      const uint32_t i4 = threadIdx.x + 256u * k;
      float4 q = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      if (4 * i4 < n) q = nlg_ld_stream_f4((const float4 *)ar + i4);
      v[4 * k] = q.x; v[4 * k + 1] = q.y; v[4 * k + 2] = q.z; v[4 * k + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < EPT; k++) {
      const uint32_t i = threadIdx.x + 256u * k;
      v[k] = i < n ? ar[i] : -INFINITY;
    }
  }
#pragma unroll
  for (int k = 0; k < EPT; k++) mx = v[k] > mx ? v[k] : mx;
  mx = nlg_block_max_f32(mx, red);
  if (first != first) mx = first;
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < EPT; k++) {
    const uint32_t i = V4 ? 4 * (threadIdx.x + 256u * (k / 4)) + (k % 4) : threadIdx.x + 256u * k;
    v[k] = expf(__fsub_rn(v[k], mx));
    if (i < n) s = __fadd_rn(s, v[k]);
  }
  s = nlg_block_sum_f32(s, red);
  if (V4) {
#pragma unroll
    for (int k = 0; k < EPT / 4; k++) {
      const uint32_t i4 = threadIdx.x + 256u * k;
      if (4 * i4 < n)
        nlg_st_stream_f4((float4 *)cr + i4,
                         make_float4(v[4 * k] / s, v[4 * k + 1] / s, v[4 * k + 2] / s, v[4 * k + 3] / s));
    }
  } else {
#pragma unroll
    for (int k = 0; k < EPT; k++) {
      const uint32_t i = threadIdx.x + 256u * k;
      if (i < n) cr[i] = v[k] / s;
    }
  }
}

// Rows too long for registers: three streaming passes, same semantics.
__global__ __launch_bounds__(256) void k_softmax_stream(const float *a, float *c, uint32_t rows,
                                                        uint32_t n) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const float *ar = a + (size_t)row * n;
  float *cr = c + (size_t)row * n;
  const float first = ar[0];
  float mx = -INFINITY;
  for (uint32_t i = threadIdx.x; i < n; i += 256) mx = ar[i] > mx ? ar[i] : mx;
  mx = nlg_block_max_f32(mx, red);
  if (first != first) mx = first;
  float s = 0.0f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) s = __fadd_rn(s, expf(__fsub_rn(ar[i], mx)));
  s = nlg_block_sum_f32(s, red);
  // each element is read by the thread that then overwrites it: in-place safe
  for (uint32_t i = threadIdx.x; i < n; i += 256) cr[i] = expf(__fsub_rn(ar[i], mx)) / s;
}

static int launch_softmax(const float *a, float *c, uint32_t rows, uint32_t n, hipStream_t st) {
  if (!rows || !n) return NLG_OK;
  const bool v4 = (n % 4 == 0) && ((((uintptr_t)a) | ((uintptr_t)c)) & 15) == 0;
  dim3 g(rows), b(256);
#define SM(EPT)                                                                  \
  do {                                                                           \
    if (v4) hipLaunchKernelGGL((k_softmax_reg<EPT, true>), g, b, 0, st, a, c, rows, n); \
    else hipLaunchKernelGGL((k_softmax_reg<EPT, false>), g, b, 0, st, a, c, rows, n);   \
  } while (0)
  if (n <= 256 * 4) SM(4);
  else if (n <= 256 * 8) SM(8);
  else if (n <= 256 * 16) SM(16);
  else if (n <= 256 * 32) SM(32);
  else hipLaunchKernelGGL(k_softmax_stream, g, b, 0, st, a, c, rows, n);
#undef SM
  NLG_LAUNCHED("softmax");
  return NLG_OK;
}

extern "C" int nlg_softmax_rows(const float *a, float *c, uint32_t rows, uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  return launch_softmax(a, c, rows, cols, nlg_stream(stream));
}

// softmax by name: A C; push (M N)
int L_softmax(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], N = p[1];
  const uint64_t rows = nlg_domain(M, groups);
  if (nlg_need(b, 0, rows * N, "softmax") || nlg_need(b, 1, rows * N, "softmax")) return NLG_ERR;
  if ((uint64_t)M * N > 0xffffffffull) return nlg_fail("softmax: M*N exceeds 2^32 elements");
  return launch_softmax((const float *)b[0].ptr, (float *)b[1].ptr, (uint32_t)rows, N, st);
}

// rmsnorm-istd (kernels.el:1249-1256): S[r] = 1/sqrt(sum(x^2)/N + 1e-6)
__global__ __launch_bounds__(256) void k_rmsnorm_istd(const float *x, float *s, uint32_t rows,
                                                      uint32_t n) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const float *xr = x + (size_t)row * n;
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) ss = __fadd_rn(ss, __fmul_rn(xr[i], xr[i]));
  ss = nlg_block_sum_f32(ss, red);
  if (threadIdx.x == 0) s[row] = 1.0f / sqrtf(__fadd_rn(ss / (float)n, EPS6));
}

int L_rmsnorm_istd(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t M = p[0], N = p[1];
  const uint64_t rows = nlg_domain(M, groups);
  if (nlg_need(b, 0, rows * N, "rmsnorm-istd") || nlg_need(b, 1, rows, "rmsnorm-istd")) return NLG_ERR;
  if (!rows) return NLG_OK;
  hipLaunchKernelGGL(k_rmsnorm_istd, dim3((uint32_t)rows), dim3(256), 0, st, (const float *)b[0].ptr,
                     (float *)b[1].ptr, (uint32_t)rows, N);
  NLG_LAUNCHED("rmsnorm-istd");
  return NLG_OK;
}

// rmsnorm-heads (kernels.el:823-842): one wave per (position, head) row.
__global__ __launch_bounds__(256) void k_rmsnorm_heads(const float *x, const float *g, float *y,
                                                       uint32_t nrows, uint32_t hd) {
  const int lane = threadIdx.x & 63;
  const uint64_t r = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= nrows) return;
  const float *xr = x + r * hd;
  float ss = 0.0f;
  for (uint32_t i = lane; i < hd; i += 64) ss = __fadd_rn(ss, __fmul_rn(xr[i], xr[i]));
  ss = nlg_wave_sum_f32(ss);
  const float inv = 1.0f / sqrtf(__fadd_rn(ss / (float)hd, EPS6));
  for (uint32_t j = lane; j < hd; j += 64) y[r * hd + j] = __fmul_rn(__fmul_rn(xr[j], inv), g[j]);
}

int L_rmsnorm_heads(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], nheads = p[1], hd = p[2];
  const uint64_t rows = nlg_domain((uint32_t)(seq * nheads), groups);
  const char *k = "rmsnorm-heads";
  if (nlg_need(b, 0, rows * hd, k) || nlg_need(b, 1, rows ? hd : 0, k) || nlg_need(b, 2, rows * hd, k))
    return NLG_ERR;
  if (!rows) return NLG_OK;
  hipLaunchKernelGGL(k_rmsnorm_heads, dim3(nlg_blocks(rows, 4)), dim3(256), 0, st,
                     (const float *)b[0].ptr, (const float *)b[1].ptr, (float *)b[2].ptr,
                     (uint32_t)rows, hd);
  NLG_LAUNCHED(k);
  return NLG_OK;
}
