// nlg_attn.hip -- attention on the reference's f32 layouts.
//
//   decode-attn / decode-attn-b (kernels.el:315-390): single-query causal GQA
//     over cached K/V.  The reference spends one invocation per output
//     element and recomputes every q.k product hd times; here a workgroup
//     owns one (sequence, head): each wave takes every 4th position, its 64
//     lanes split the head dimension (coalesced 512-byte K/V rows at hd=128),
//     the q.k product is one DPP reduction, and the four waves' running
//     (z, ctx) are merged through LDS.
//   attn-causal-gqa (kernels.el:934-990): one wave per (head, query).
//   attn-scores / attn-context (kernels.el:205-235): per element, serial in
//     the reference's order (bit-identical up to the 1/sqrt(hd) scale).
// Every access is bounds-checked (reads past a buffer give 0, writes are
// dropped) because POS comes from device memory.
#include <math.h>

#include "nlg_internal.h"

#define NEG_BIG (-1.0e30f)

struct AB {
  const float *p;
  uint32_t n;
};
__device__ __forceinline__ float ald(const AB &b, uint32_t i) { return i < b.n ? b.p[i] : 0.0f; }

struct DecArgs {
  AB q, ck, cv, pos;
  float *c;
  uint32_t nc;
  uint32_t B, dim, heads, kvheads, maxseq, hd, grp, kvdim;
  uint32_t hslots;  // head slots per sequence = ceil(dim / hd)
  uint32_t domain;  // output elements that are written: min(B*dim, 64*groups)
};

// EPL: head elements per lane (hd <= 64*EPL).
template <int EPL>
__global__ __launch_bounds__(256) void k_decode_attn(DecArgs a) {
  __shared__ float s_ctx[4][64 * EPL];
  __shared__ float s_z[4], s_mx[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t bb = blockIdx.x / a.hslots, h = blockIdx.x % a.hslots;
  const uint32_t kvh = a.grp ? h / a.grp : 0u;
  const uint32_t pos = nlg_f2u(ald(a.pos, 0)), len = pos + 1u;
  const uint32_t cbase = (bb * a.maxseq) * a.kvdim, c0q = bb * a.dim + h * a.hd;
  const float coef = 1.0f / sqrtf((float)a.hd);
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const uint32_t t = lane + 64 * e;
    q[e] = t < a.hd ? ald(a.q, c0q + t) : 0.0f;
  }
  // Positions whose K row starts past both cache buffers read as all-zero
  // rows: score exactly 0 and a zero V row.  They are folded in analytically
  // so a wild POS cannot make the loop run for billions of trips.
  const uint32_t kvoff = kvh * a.hd;
  uint64_t lim = a.ck.n > a.cv.n ? a.ck.n : a.cv.n;
  uint64_t jloop64 = len;
  if (a.kvdim) {
    uint64_t base0 = (uint64_t)cbase + kvoff;
    uint64_t jmax = base0 >= lim ? 0 : (lim - base0 + a.kvdim - 1) / a.kvdim;
    if (jloop64 > jmax) jloop64 = jmax;
  }
  const uint32_t jloop = (uint32_t)jloop64;
  // pass 1: the maximum score (seeded -1e30 as the reference)
  float mx = NEG_BIG;
  for (uint32_t j = w; j < jloop; j += 4) {
    const uint32_t kb = cbase + (j * a.kvdim + kvoff);
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      if (t < a.hd) d = __fadd_rn(d, __fmul_rn(q[e], ald(a.ck, kb + t)));
    }
    const float s = __fmul_rn(nlg_wave_sum_f32(d), coef);
    if (s > mx) mx = s;
  }
  if (jloop < len && 0.0f > mx) mx = 0.0f;
  if (lane == 0) s_mx[w] = mx;
  __syncthreads();
  mx = s_mx[0];
  for (int i = 1; i < 4; i++) mx = s_mx[i] > mx ? s_mx[i] : mx;
  // pass 2: z and ctx
  float z = 0.0f, ctx[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) ctx[e] = 0.0f;
  for (uint32_t j = w; j < jloop; j += 4) {
    const uint32_t kb = cbase + (j * a.kvdim + kvoff);
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      if (t < a.hd) d = __fadd_rn(d, __fmul_rn(q[e], ald(a.ck, kb + t)));
    }
    const float ee = expf(__fsub_rn(__fmul_rn(nlg_wave_sum_f32(d), coef), mx));
    z = __fadd_rn(z, ee);
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      if (t < a.hd) ctx[e] = __fadd_rn(ctx[e], __fmul_rn(ee, ald(a.cv, kb + t)));
    }
  }
#pragma unroll
  for (int e = 0; e < EPL; e++) s_ctx[w][lane + 64 * e] = ctx[e];
  if (lane == 0) s_z[w] = z;
  __syncthreads();
  if (w == 0) {
    float zt = __fadd_rn(__fadd_rn(s_z[0], s_z[1]), __fadd_rn(s_z[2], s_z[3]));
    if (jloop < len) zt = __fadd_rn(zt, __fmul_rn((float)(len - jloop), expf(__fsub_rn(0.0f, mx))));
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      const float ct = __fadd_rn(__fadd_rn(s_ctx[0][t], s_ctx[1][t]), __fadd_rn(s_ctx[2][t], s_ctx[3][t]));
      const uint32_t oc = h * a.hd + t;  // output column within the sequence
      const uint32_t idx = bb * a.dim + oc;
      if (t < a.hd && oc < a.dim && idx < a.domain && idx < a.nc) a.c[idx] = ct / zt;
    }
  }
}

static int decode_attn_common(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st,
                              bool batched) {
  DecArgs a;
  a.B = batched ? p[0] : 1u;
  a.dim = p[batched ? 1 : 0];
  a.heads = p[batched ? 2 : 1];
  a.kvheads = p[batched ? 3 : 2];
  a.maxseq = batched ? p[4] : 0u;
  const char *k = batched ? "decode-attn-b" : "decode-attn";
  if (!a.heads || !a.kvheads) return nlg_fail("%s: heads and kvheads must be nonzero", k);
  a.hd = a.dim / a.heads;
  a.grp = a.heads / a.kvheads;
  a.kvdim = a.kvheads * a.hd;
  if (!a.hd) return NLG_OK;  // the reference divides by zero only inside an empty domain
  if (a.hd > 512) return nlg_fail("%s: head dim %u > 512", k, a.hd);
  a.hslots = (a.dim + a.hd - 1) / a.hd;
  const uint64_t dom = nlg_domain((uint32_t)(a.B * a.dim), groups);
  if (!dom) return NLG_OK;
  a.domain = (uint32_t)dom;
  a.q = AB{(const float *)b[0].ptr, b[0].nfloats};
  a.ck = AB{(const float *)b[1].ptr, b[1].nfloats};
  a.cv = AB{(const float *)b[2].ptr, b[2].nfloats};
  a.pos = AB{(const float *)b[3].ptr, b[3].nfloats};
  a.c = (float *)b[4].ptr;
  a.nc = b[4].nfloats;
  const uint32_t seqs = (uint32_t)((dom + a.dim - 1) / a.dim);
  dim3 g(seqs * a.hslots), blk(256);
  if (a.hd <= 64) hipLaunchKernelGGL(k_decode_attn<1>, g, blk, 0, st, a);
  else if (a.hd <= 128) hipLaunchKernelGGL(k_decode_attn<2>, g, blk, 0, st, a);
  else if (a.hd <= 256) hipLaunchKernelGGL(k_decode_attn<4>, g, blk, 0, st, a);
  else hipLaunchKernelGGL(k_decode_attn<8>, g, blk, 0, st, a);
  NLG_LAUNCHED(k);
  return NLG_OK;
}
int L_decode_attn(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return decode_attn_common(b, p, groups, st, false);
}
int L_decode_attn_b(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return decode_attn_common(b, p, groups, st, true);
}

// attn-causal-gqa: one wave per (head, query i), lanes over the head dim.
struct GqaArgs {
  AB q, k, v;
  float *ctx;
  uint32_t nctx;
  uint32_t seq, heads, kvheads, hd, n;  // n = rows handled: min(heads*seq, 64*groups)
};
template <int EPL>
__global__ __launch_bounds__(256) void k_attn_gqa(GqaArgs a) {
  const int lane = threadIdx.x & 63;
  const uint64_t r = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.n) return;
  const uint32_t idx = (uint32_t)r, h = idx / a.seq, i = idx % a.seq;
  const uint32_t qdim = a.heads * a.hd, kvdim = a.kvheads * a.hd, grp = a.heads / a.kvheads;
  const uint32_t qb = i * qdim + h * a.hd, kc = (grp ? h / grp : 0u) * a.hd;
  const float scale = 1.0f / sqrtf((float)a.hd);
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const uint32_t t = lane + 64 * e;
    q[e] = t < a.hd ? ald(a.q, qb + t) : 0.0f;
  }
  const uint32_t n = i + 1;
  float mx = NEG_BIG;
  for (uint32_t j = 0; j < n; j++) {
    const uint32_t kb = j * kvdim + kc;
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      if (t < a.hd) d = __fadd_rn(d, __fmul_rn(q[e], ald(a.k, kb + t)));
    }
    const float s = __fmul_rn(nlg_wave_sum_f32(d), scale);
    if (s > mx) mx = s;
  }
  float sm = 0.0f, ctx[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) ctx[e] = 0.0f;
  for (uint32_t j = 0; j < n; j++) {
    const uint32_t kb = j * kvdim + kc;
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      if (t < a.hd) d = __fadd_rn(d, __fmul_rn(q[e], ald(a.k, kb + t)));
    }
    const float ee = expf(__fsub_rn(__fmul_rn(nlg_wave_sum_f32(d), scale), mx));
    sm = __fadd_rn(sm, ee);
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const uint32_t t = lane + 64 * e;
      if (t < a.hd) ctx[e] = __fadd_rn(ctx[e], __fmul_rn(ee, ald(a.v, kb + t)));
    }
  }
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const uint32_t t = lane + 64 * e;
    if (t < a.hd && qb + t < a.nctx) a.ctx[qb + t] = ctx[e] / sm;
  }
}

int L_attn_causal_gqa(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  GqaArgs a;
  a.seq = p[0];
  a.heads = p[1];
  a.kvheads = p[2];
  a.hd = p[3];
  if (!a.kvheads || !a.seq) return a.seq ? nlg_fail("attn-causal-gqa: kvheads must be nonzero") : NLG_OK;
  if (a.hd > 512) return nlg_fail("attn-causal-gqa: head dim %u > 512", a.hd);
  const uint64_t n = nlg_domain((uint32_t)(a.heads * a.seq), groups);
  if (!n || !a.hd) return NLG_OK;
  a.n = (uint32_t)n;
  a.q = AB{(const float *)b[0].ptr, b[0].nfloats};
  a.k = AB{(const float *)b[1].ptr, b[1].nfloats};
  a.v = AB{(const float *)b[2].ptr, b[2].nfloats};
  a.ctx = (float *)b[3].ptr;
  a.nctx = b[3].nfloats;
  dim3 g(nlg_blocks(n, 4)), blk(256);
  if (a.hd <= 64) hipLaunchKernelGGL(k_attn_gqa<1>, g, blk, 0, st, a);
  else if (a.hd <= 128) hipLaunchKernelGGL(k_attn_gqa<2>, g, blk, 0, st, a);
  else if (a.hd <= 256) hipLaunchKernelGGL(k_attn_gqa<4>, g, blk, 0, st, a);
  else hipLaunchKernelGGL(k_attn_gqa<8>, g, blk, 0, st, a);
  NLG_LAUNCHED("attn-causal-gqa");
  return NLG_OK;
}

// attn-scores (kernels.el:205-222), per element, serial dot in reference order.
__global__ __launch_bounds__(256) void k_attn_scores(AB q, AB k, float *s, uint32_t ns, uint32_t n,
                                                     uint32_t seq, uint32_t dim, uint32_t heads,
                                                     uint32_t kvheads) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const uint32_t hd = dim / heads, grp = heads / kvheads, kvdim = kvheads * hd;
  const uint32_t h = idx / (seq * seq), rem = idx % (seq * seq), i = rem / seq, j = rem % seq;
  if (j > i && idx < ns) s[idx] = NEG_BIG;
  if (j < i + 1) {
    const uint32_t kvh = grp ? h / grp : 0u, qb = i * dim + h * hd, kb = j * kvdim + kvh * hd;
    float acc = 0.0f;
    for (uint32_t t = 0; t < hd; t++) acc = __fadd_rn(acc, __fmul_rn(ald(q, qb + t), ald(k, kb + t)));
    if (idx < ns) s[idx] = __fmul_rn(acc, 1.0f / sqrtf((float)hd));
  }
}
int L_attn_scores(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], dim = p[1], heads = p[2], kvheads = p[3];
  if (!heads || !kvheads) return nlg_fail("attn-scores: heads and kvheads must be nonzero");
  const uint64_t n = nlg_domain((uint32_t)((heads * seq) * seq), groups);
  if (!n || !seq) return NLG_OK;
  hipLaunchKernelGGL(k_attn_scores, dim3(nlg_blocks(n, 256)), dim3(256), 0, st,
                     AB{(const float *)b[0].ptr, b[0].nfloats}, AB{(const float *)b[1].ptr, b[1].nfloats},
                     (float *)b[2].ptr, b[2].nfloats, (uint32_t)n, seq, dim, heads, kvheads);
  NLG_LAUNCHED("attn-scores");
  return NLG_OK;
}

// attn-context (kernels.el:223-235), per element, serial in reference order.
__global__ __launch_bounds__(256) void k_attn_context(AB pm, AB v, float *c, uint32_t nc, uint32_t n,
                                                      uint32_t seq, uint32_t dim, uint32_t heads,
                                                      uint32_t kvheads) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const uint32_t hd = dim / heads, grp = heads / kvheads, kvdim = kvheads * hd;
  const uint32_t i = idx / dim, cc = idx % dim;
  const uint32_t h = hd ? cc / hd : 0u, t = hd ? cc % hd : 0u, kvh = grp ? h / grp : 0u;
  const uint32_t pb = h * (seq * seq) + i * seq;
  float acc = 0.0f;
  for (uint32_t j = 0; j < seq; j++)
    acc = __fadd_rn(acc, __fmul_rn(ald(pm, pb + j), ald(v, j * kvdim + (kvh * hd + t))));
  if (idx < nc) c[idx] = acc;
}
int L_attn_context(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  const uint32_t seq = p[0], dim = p[1], heads = p[2], kvheads = p[3];
  if (!heads || !kvheads) return nlg_fail("attn-context: heads and kvheads must be nonzero");
  const uint64_t n = nlg_domain((uint32_t)(seq * dim), groups);
  if (!n) return NLG_OK;
  hipLaunchKernelGGL(k_attn_context, dim3(nlg_blocks(n, 256)), dim3(256), 0, st,
                     AB{(const float *)b[0].ptr, b[0].nfloats}, AB{(const float *)b[1].ptr, b[1].nfloats},
                     (float *)b[2].ptr, b[2].nfloats, (uint32_t)n, seq, dim, heads, kvheads);
  NLG_LAUNCHED("attn-context");
  return NLG_OK;
}
