// Causal GQA attention for a whole prompt on the matrix cores.
//
// Semantics: attn-causal-gqa (kernels.el:934-990) over the fp16 K/V cache
// the decode path uses ([seq][kvheads][max_seq][head_dim]): query row r is
// sequence r / qper at position p = pos[0] + r % qper and attends positions
// 0..p of its sequence with s = (q.k)/sqrt(head_dim), e = exp(s - max),
// ctx = sum(e v) / sum(e), accumulated in f32.
//
// A workgroup takes 32 query positions of one sequence and one kv head, one
// wave per query head of the group, so each K/V block is staged in LDS once
// for all of them.  Per block of 32 keys a wave computes S^T = K Q^T (32 keys
// x 32 queries) with v_mfma_f32_32x32x16_f16, whose layout, checked on
// gfx950, is C[i][j] = sum over lane groups g = 0..1 and elements e < 8 of
// A[lane 32g + i][e] * B[lane 32g + j][e], lane l's result r at row
// (r % 4) + 8 (r / 4) + 4 (l / 32), column l % 32.  That leaves each lane
// with one query's 16 scores, so the online softmax (running max and sum,
// rescaling the context) needs one exchange with lane l ^ 32, and the
// probabilities are already the B operand of O^T += V^T P^T (their keys in
// the order the score layout gives them; V^T is read from a transposed LDS
// copy in the same order).  Q and P enter the f16 matrix cores as hi + lo
// halves (x = hi + lo exactly to 22 bits), so the products carry f32-grade
// precision; K and V are fp16 already.

#include "nlg_internal.h"

#include <math.h>

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct PrefillArgs {
  const float *q;
  const uint16_t *kc, *vc;
  const int32_t *pos;
  float *ctx;
  uint32_t qper, heads, kvheads, max_seq, nq;
  float coef;  // 1/sqrt(head_dim)
};

#define PA_KB 32  // keys per block
#define PA_QB 32  // query positions per workgroup

__device__ __forceinline__ v8h f16x8(uint4 u) { return __builtin_bit_cast(v8h, u); }

template <int HD, int GRP>
__global__ __launch_bounds__(64 * GRP, GRP >= 4 ? 8 / GRP : 1) void k_prefill_attn(PrefillArgs a) {
  constexpr int NT = 64 * GRP;
  constexpr int KP = HD + 8;       // K row pitch in halves (staggers the banks)
  constexpr int VP = PA_KB + 4;    // transposed-V row pitch in halves
  constexpr int KI = (PA_KB * HD / 8 + NT - 1) / NT;   // 16-byte K pieces per thread
  constexpr int VI = (PA_KB / 4 * HD / 4 + NT - 1) / NT;  // 4x4 V tiles per thread
  __shared__ __align__(16) uint16_t s_k[2][PA_KB * KP];
  __shared__ __align__(16) uint16_t s_v[2][HD * VP];
  asm volatile("" ::"s"(a.q), "s"(a.kc), "s"(a.vc), "s"(a.pos), "s"(a.ctx), "s"(a.qper), "s"(a.kvheads),
               "s"(a.max_seq), "s"(a.nq), "s"(a.coef));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 31, lg = lane >> 5;
  const uint32_t kvh = blockIdx.y, sq = blockIdx.z, head = kvh * GRP + w;
  const int32_t pos0 = a.pos[0];
  // this lane's query: prompt row i (clamped for the tail block)
  const uint32_t i = blockIdx.x * PA_QB + li;
  const bool live = i < a.qper;
  const uint32_t ic = live ? i : a.qper - 1;
  const uint32_t row = sq * a.qper + ic;
  const int32_t pj = pos0 + (int32_t)ic;
  const uint32_t ilast = min(blockIdx.x * PA_QB + PA_QB - 1, a.qper - 1);
  const int32_t plast = min(pos0 + (int32_t)ilast, (int32_t)a.max_seq - 1);
  const uint32_t nkb = plast < 0 ? 0u : (uint32_t)plast / PA_KB + 1;
  const size_t cache0 = (size_t)(sq * a.kvheads + kvh) * a.max_seq * HD;
  const uint16_t *kb0 = a.kc + cache0, *vb0 = a.vc + cache0;
  const uint32_t klast = a.max_seq - 1;

  // K block: piece t = key t / (HD/8), 8 halves at (t % (HD/8)) * 8.
  // V block: tile t = 4 keys 4 (t / (HD/4)) .. +3 x 4 dims 4 (t % (HD/4)) .. +3.
  // staging registers as vectors (arrays assigned under a branch go to scratch)
  typedef uint32_t kvec __attribute__((ext_vector_type(4 * KI)));
  typedef uint32_t vvec __attribute__((ext_vector_type(8 * VI)));
  kvec kr;
  vvec vr;
#define PA_LOAD(kb)                                                                       \
  do {                                                                                    \
    _Pragma("unroll") for (int u = 0; u < KI; u++) {                                      \
      const uint32_t t = threadIdx.x + NT * u;                                            \
      const uint32_t key = min((kb) * PA_KB + t / (HD / 8), klast);                        \
      if ((PA_KB * HD / 8) % NT == 0 || t < PA_KB * HD / 8) {                             \
        const uint4 x = *(const uint4 *)(kb0 + (size_t)key * HD + 8 * (t % (HD / 8)));     \
        kr[4 * u] = x.x; kr[4 * u + 1] = x.y; kr[4 * u + 2] = x.z; kr[4 * u + 3] = x.w;     \
      }                                                                                   \
    }                                                                                     \
    _Pragma("unroll") for (int u = 0; u < VI; u++) {                                      \
      const uint32_t t = threadIdx.x + NT * u;                                            \
      _Pragma("unroll") for (int e = 0; e < 4; e++) {                                     \
        const uint32_t key = min((kb) * PA_KB + 4 * (t / (HD / 4)) + e, klast);            \
        if ((PA_KB / 4 * HD / 4) % NT == 0 || t < PA_KB / 4 * HD / 4) {                   \
          const uint2 x = *(const uint2 *)(vb0 + (size_t)key * HD + 4 * (t % (HD / 4)));   \
          vr[8 * u + 2 * e] = x.x; vr[8 * u + 2 * e + 1] = x.y;                           \
        }                                                                                 \
      }                                                                                   \
    }                                                                                     \
  } while (0)
#define PA_STORE(buf)                                                                     \
  do {                                                                                    \
    _Pragma("unroll") for (int u = 0; u < KI; u++) {                                      \
      const uint32_t t = threadIdx.x + NT * u;                                            \
      if ((PA_KB * HD / 8) % NT == 0 || t < PA_KB * HD / 8)                               \
        *(uint4 *)(&s_k[buf][(t / (HD / 8)) * KP + 8 * (t % (HD / 8))]) =                  \
            make_uint4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]);              \
    }                                                                                     \
    _Pragma("unroll") for (int u = 0; u < VI; u++) {                                      \
      const uint32_t t = threadIdx.x + NT * u;                                            \
      if ((PA_KB / 4 * HD / 4) % NT == 0 || t < PA_KB / 4 * HD / 4) {                                                       \
        const uint32_t k4 = 4 * (t / (HD / 4)), d4 = 4 * (t % (HD / 4));                  \
        /* dims d4 + c: the 4 keys' halves c, low key first */                            \
        _Pragma("unroll") for (int c = 0; c < 4; c++) {                                   \
          const int sh = 16 * (c & 1);                                                    \
          const uint32_t h0 = (vr[8 * u + 0 + c / 2] >> sh) & 0xffffu;                    \
          const uint32_t h1 = (vr[8 * u + 2 + c / 2] >> sh) & 0xffffu;                    \
          const uint32_t h2 = (vr[8 * u + 4 + c / 2] >> sh) & 0xffffu;                    \
          const uint32_t h3 = (vr[8 * u + 6 + c / 2] >> sh) & 0xffffu;                    \
          *(uint2 *)(&s_v[buf][(d4 + c) * VP + k4]) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16)); \
        }                                                                                 \
      }                                                                                   \
    }                                                                                     \
  } while (0)

  // Q as hi + lo halves: lane (lg, li) holds dims 16 s + 8 lg + 0..7 of its query
  v8h qh[HD / 16], ql[HD / 16];
  {
    const float *qp = a.q + (size_t)row * a.nq + (size_t)head * HD + 8 * lg;
#pragma unroll
    for (int s = 0; s < HD / 16; s++) {
      typedef float v8f __attribute__((ext_vector_type(8)));
      const v8f x = *(const v8f *)(qp + 16 * s);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const _Float16 h = (_Float16)x[e];
        qh[s][e] = h;
        ql[s][e] = (_Float16)(x[e] - (float)h);
      }
    }
  }
  v16f o[HD / 32];
#pragma unroll
  for (int t = 0; t < HD / 32; t++) o[t] = (v16f){};
  float m = -1.0e30f, l = 0.0f;
  if (nkb) {
    PA_LOAD(0u);
    PA_STORE(0);
  }
  for (uint32_t kb = 0; kb < nkb; kb++) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) PA_LOAD(kb + 1);
    __syncthreads();
    // S^T = K Q^T: lane (lg, li) gets keys 32 kb + 8 (r/4) + 4 lg + r%4 of query li
    v16f sc = {};
#pragma unroll
    for (int s = 0; s < HD / 16; s++) {
      const v8h kf = f16x8(*(const uint4 *)(&s_k[buf][li * KP + 16 * s + 8 * lg]));
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qh[s], sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, ql[s], sc, 0, 0, 0);
    }
    float mb = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int32_t key = (int32_t)(kb * PA_KB + 8 * (r / 4) + 4 * lg + r % 4);
      sc[r] = key <= pj ? sc[r] * a.coef : -INFINITY;
      mb = fmaxf(mb, sc[r]);
    }
    mb = fmaxf(mb, __shfl_xor(mb, 32));
    const float mn = fmaxf(m, mb);
    const float al = expf(m - mn);
    float ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      sc[r] = expf(sc[r] - mn);
      ls += sc[r];
    }
    ls += __shfl_xor(ls, 32);
    l = l * al + ls;
    m = mn;
#pragma unroll
    for (int t = 0; t < HD / 32; t++) o[t] *= al;
    // O^T += V^T P^T over two steps of 16 keys; element e of step s2 is key
    // 16 s2 + 8 (e/4) + 4 lg + e%4 in both operands
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      v8h ph, pl;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const _Float16 h = (_Float16)sc[8 * s2 + e];
        ph[e] = h;
        pl[e] = (_Float16)(sc[8 * s2 + e] - (float)h);
      }
#pragma unroll
      for (int t = 0; t < HD / 32; t++) {
        const uint16_t *vrow = &s_v[buf][(32 * t + li) * VP + 16 * s2 + 4 * lg];
        const uint2 va = *(const uint2 *)vrow, vb = *(const uint2 *)(vrow + 8);
        const v8h vf = f16x8(make_uint4(va.x, va.y, vb.x, vb.y));
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, ph, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pl, o[t], 0, 0, 0);
      }
    }
    if (kb + 1 < nkb) PA_STORE(buf ^ 1);
  }
#undef PA_LOAD
#undef PA_STORE
  // O^T tile t, register r: dim 32 t + 8 (r/4) + 4 lg + r%4 of query li
  if (live) {
    float *cp = a.ctx + (size_t)row * a.nq + (size_t)head * HD + 4 * lg;
#pragma unroll
    for (int t = 0; t < HD / 32; t++) {
#pragma unroll
      for (int rq = 0; rq < 4; rq++) {
        float4 v;
        v.x = l > 0.0f ? o[t][4 * rq] / l : 0.0f;
        v.y = l > 0.0f ? o[t][4 * rq + 1] / l : 0.0f;
        v.z = l > 0.0f ? o[t][4 * rq + 2] / l : 0.0f;
        v.w = l > 0.0f ? o[t][4 * rq + 3] / l : 0.0f;
        *(float4 *)(cp + 32 * t + 8 * rq) = v;
      }
    }
  }
}

}  // namespace

int nlg_prefill_attn(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos, uint32_t rows,
                     uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                     float *ctx, hipStream_t st) {
  if (!rows) return NLG_OK;
  if (!q || !kc || !vc || !pos || !ctx) return nlg_fail("prefill attn: null pointer");
  if (head_dim != 64 && head_dim != 128) return nlg_fail("prefill attn: head_dim %u not 64 or 128", head_dim);
  if (!kvheads || heads % kvheads) return nlg_fail("prefill attn: heads %u not a multiple of kv heads %u", heads, kvheads);
  const uint32_t grp = heads / kvheads;
  if (grp != 1 && grp != 2 && grp != 4 && grp != 8) return nlg_fail("prefill attn: heads/kvheads %u not 1, 2, 4 or 8", grp);
  if (!qper || rows % qper) return nlg_fail("prefill attn: rows %u not a multiple of rows per sequence %u", rows, qper);
  if (!max_seq) return nlg_fail("prefill attn: max_seq is 0");
  if (((uintptr_t)q & 15) || ((uintptr_t)kc & 15) || ((uintptr_t)vc & 15) || ((uintptr_t)ctx & 15))
    return nlg_fail("prefill attn: q, caches and ctx must be 16-byte aligned");
  const uint32_t nseq = rows / qper;
  if (nseq > 65535 || kvheads > 65535) return nlg_fail("prefill attn: too many sequences or kv heads");
  PrefillArgs a{q, kc, vc, pos, ctx, qper, heads, kvheads, max_seq, heads * head_dim,
                1.0f / sqrtf((float)head_dim)};  // (/ 1.0 (sqrt (float hd)))
  const dim3 grid((qper + PA_QB - 1) / PA_QB, kvheads, nseq), blk(64 * grp);
#define PA(HD)                                                                             \
  do {                                                                                     \
    if (grp == 1) hipLaunchKernelGGL((k_prefill_attn<HD, 1>), grid, blk, 0, st, a);        \
    else if (grp == 2) hipLaunchKernelGGL((k_prefill_attn<HD, 2>), grid, blk, 0, st, a);   \
    else if (grp == 4) hipLaunchKernelGGL((k_prefill_attn<HD, 4>), grid, blk, 0, st, a);   \
    else hipLaunchKernelGGL((k_prefill_attn<HD, 8>), grid, blk, 0, st, a);                 \
  } while (0)
  if (head_dim == 128) PA(128); else PA(64);
#undef PA
  NLG_LAUNCHED("prefill attention (fp16 KV, MFMA)");
  return NLG_OK;
}

extern "C" int nlg_prefill_attn_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                    const int32_t *pos, uint32_t rows, uint32_t qper, uint32_t heads,
                                    uint32_t kvheads, uint32_t head_dim, uint32_t max_seq, float *ctx,
                                    void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  return nlg_prefill_attn(q, kcache, vcache, pos, rows, qper, heads, kvheads, head_dim, max_seq, ctx,
                          nlg_stream(stream));
}
