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
// precision; K and V are fp16 already.  Scores are kept in base 2 (log2 e
// folded into the 1/sqrt(hd) scale), so every exponential is one v_exp_f32
// instead of a correctly rounded expf.

#include "nlg_internal.h"
#include "nlg_quant.h"

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
  float coef;  // log2(e)/sqrt(head_dim): scores in base 2
  // key-range split (SPLIT kernels): workgroup x = query block x / maxp,
  // piece x % maxp of kps key blocks; each piece leaves its unnormalised
  // context [piece][row][nq] and (max, sum) [piece][row][heads][2] for
  // k_prefill_merge
  float *part_o, *part_ml;
  uint32_t kps, maxp;
};

#define PA_KB 32  // keys per block
#define PA_QB 32  // query positions per workgroup

__device__ __forceinline__ v8h f16x8(uint4 u) { return __builtin_bit_cast(v8h, u); }

// The lo halves of two probabilities, x - hi rounded to f16 (hi = x rounded
// to f16, the halves of h2), packed: one mixed-precision FMA each, x * 1 - hi
// in f32 (exact: hi is x's nearest f16) rounded once -- the value the
// convert / subtract / convert chain gives, in a third of the instructions.
__device__ __forceinline__ uint32_t pa_lo2(float x0, float x1, uint32_t h2) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(r) : "v"(x0), "v"(h2));
  asm("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(r) : "v"(x1), "v"(h2));
  return r;
}

template <int HD, int GRP, bool SPLIT>
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
  const uint32_t qb = SPLIT ? blockIdx.x / a.maxp : blockIdx.x, piece = SPLIT ? blockIdx.x % a.maxp : 0;
  const int32_t pos0 = a.pos[0];
  // this lane's query: prompt row i (clamped for the tail block)
  const uint32_t i = qb * PA_QB + li;
  const bool live = i < a.qper;
  const uint32_t ic = live ? i : a.qper - 1;
  const uint32_t row = sq * a.qper + ic;
  const int32_t pj = pos0 + (int32_t)ic;
  const uint32_t ilast = min(qb * PA_QB + PA_QB - 1, a.qper - 1);
  const int32_t plast = min(pos0 + (int32_t)ilast, (int32_t)a.max_seq - 1);
  const uint32_t nkb_all = plast < 0 ? 0u : (uint32_t)plast / PA_KB + 1;
  // this workgroup's key blocks: [kbf, nkb)
  const uint32_t kbf = SPLIT ? min(piece * a.kps, nkb_all) : 0u;
  const uint32_t nkb = SPLIT ? min(kbf + a.kps, nkb_all) : nkb_all;
  if (SPLIT && kbf >= nkb && piece) return;  // past the causal range (piece 0 always reports)
  const size_t cache0 = (size_t)(sq * a.kvheads + kvh) * a.max_seq * HD;
  const uint16_t *kb0 = a.kc + cache0, *vb0 = a.vc + cache0;

  // Block kb's rows through a buffer resource starting at its first row
  // (scalar arithmetic only): each thread's offset in a block is fixed, and
  // rows past the cache read 0 -- never attended: their scores are masked
  // and their V rows zeroed below.
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  typedef uint32_t v2u __attribute__((ext_vector_type(2)));
#define PA_RES(base, kb) nlg_buffer_rsrc((base) + (size_t)(kb) * PA_KB * HD, (a.max_seq - (kb) * PA_KB) * HD * 2u)
  // K block: piece t = key t / (HD/8), 8 halves at (t % (HD/8)) * 8.
  // V block: tile t = 4 keys 4 (t / (HD/4)) .. +3 x 4 dims 4 (t % (HD/4)) .. +3.
  // staging registers as vectors (arrays assigned under a branch go to scratch)
  typedef uint32_t kvec __attribute__((ext_vector_type(4 * KI)));
  typedef uint32_t vvec __attribute__((ext_vector_type(8 * VI)));
  kvec kr;
  vvec vr;
#define PA_LOAD(kb)                                                                       \
  do {                                                                                    \
    const __amdgpu_buffer_rsrc_t kres = PA_RES(kb0, kb), vres = PA_RES(vb0, kb);          \
    _Pragma("unroll") for (int u = 0; u < KI; u++) {                                      \
      const uint32_t t = threadIdx.x + NT * u;                                            \
      if ((PA_KB * HD / 8) % NT == 0 || t < PA_KB * HD / 8) {                             \
        const v4u x = __builtin_amdgcn_raw_buffer_load_b128(                              \
            kres, (int)(2 * ((t / (HD / 8)) * HD + 8 * (t % (HD / 8)))), 0, 0);             \
        kr[4 * u] = x.x; kr[4 * u + 1] = x.y; kr[4 * u + 2] = x.z; kr[4 * u + 3] = x.w;     \
      }                                                                                   \
    }                                                                                     \
    _Pragma("unroll") for (int u = 0; u < VI; u++) {                                      \
      const uint32_t t = threadIdx.x + NT * u;                                            \
      _Pragma("unroll") for (int e = 0; e < 4; e++) {                                     \
        if ((PA_KB / 4 * HD / 4) % NT == 0 || t < PA_KB / 4 * HD / 4) {                   \
          const v2u x = __builtin_amdgcn_raw_buffer_load_b64(                             \
              vres, (int)(2 * ((4 * (t / (HD / 4)) + e) * HD + 4 * (t % (HD / 4)))), 0, 0); \
          vr[8 * u + 2 * e] = x.x; vr[8 * u + 2 * e + 1] = x.y;                           \
        }                                                                                 \
      }                                                                                   \
    }                                                                                     \
  } while (0)
#define PA_STORE(buf, kb)                                                                 \
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
        /* keys past plast (never attended here; the cache may hold anything  */         \
        /* there, NaN included, and 0 x NaN is NaN) go in as zeros            */         \
        const int32_t kk = (int32_t)((kb) * PA_KB + k4);                                   \
        const uint32_t m0 = kk <= plast ? 0xffffu : 0u, m1 = kk + 1 <= plast ? 0xffffu : 0u; \
        const uint32_t m2 = kk + 2 <= plast ? 0xffffu : 0u, m3 = kk + 3 <= plast ? 0xffffu : 0u; \
        /* dims d4 + c: the 4 keys' halves c, low key first (a block wholly */          \
        /* inside the prompt pairs them with byte permutes, nothing to zero) */           \
        if ((int32_t)((kb) * PA_KB + PA_KB - 1) <= plast) {                               \
          _Pragma("unroll") for (int c = 0; c < 4; c++) {                                 \
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;                     \
            *(uint2 *)(&s_v[buf][(d4 + c) * VP + k4]) =                                   \
                make_uint2(__builtin_amdgcn_perm(vr[8 * u + 2 + c / 2], vr[8 * u + 0 + c / 2], sel), \
                           __builtin_amdgcn_perm(vr[8 * u + 6 + c / 2], vr[8 * u + 4 + c / 2], sel)); \
          }                                                                               \
        } else {                                                                          \
          _Pragma("unroll") for (int c = 0; c < 4; c++) {                                 \
            const int sh = 16 * (c & 1);                                                  \
            const uint32_t h0 = (vr[8 * u + 0 + c / 2] >> sh) & m0;                       \
            const uint32_t h1 = (vr[8 * u + 2 + c / 2] >> sh) & m1;                       \
            const uint32_t h2 = (vr[8 * u + 4 + c / 2] >> sh) & m2;                       \
            const uint32_t h3 = (vr[8 * u + 6 + c / 2] >> sh) & m3;                       \
            *(uint2 *)(&s_v[buf][(d4 + c) * VP + k4]) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16)); \
          }                                                                               \
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
  if (nkb > kbf) {
    PA_LOAD(kbf);
    PA_STORE(kbf & 1, kbf);
  }
  for (uint32_t kb = kbf; kb < nkb; kb++) {
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
    // (q.k / sqrt(hd)) * log2(e); keys past the lane's query masked, which
    // only the blocks that reach past the block's first query need
    float mb = -INFINITY;
    if ((int32_t)(kb * PA_KB + PA_KB - 1) <= pos0 + (int32_t)(qb * PA_QB)) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        sc[r] = sc[r] * a.coef;
        mb = fmaxf(mb, sc[r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int32_t key = (int32_t)(kb * PA_KB + 8 * (r / 4) + 4 * lg + r % 4);
        sc[r] = key <= pj ? sc[r] * a.coef : -INFINITY;
        mb = fmaxf(mb, sc[r]);
      }
    }
    // lanes l and l ^ 32 hold the same query: v_permlane32_swap hands each
    // the other's value (the pair it returns is {x[l], x[l ^ 32]})
    {
      const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
      mb = fmaxf(__uint_as_float(pr[0]), __uint_as_float(pr[1]));
    }
    // The running reference m moves only when a block beats it by more than
    // 2^8 (probabilities then stay <= 256, which the fp16 hi + lo split
    // carries exactly), so most blocks skip rescaling the context: the
    // multiplies run only when some query of the wave moved.
    const bool up = mb > m + 8.0f;
    const float mn = up ? mb : m;
    const float al = nlg_exp2(m - mn);  // 1 where m stays
    float ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      sc[r] = nlg_exp2(sc[r] - mn);
      ls += sc[r];
    }
    {
      const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(ls), __float_as_uint(ls), false, false);
      ls = __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
    }
    l = l * al + ls;
    m = mn;
    if (__builtin_amdgcn_ballot_w64(up) != 0ull) {
#pragma unroll
      for (int t = 0; t < HD / 32; t++) o[t] *= al;
    }
    // O^T += V^T P^T over two steps of 16 keys; element e of step s2 is key
    // 16 s2 + 8 (e/4) + 4 lg + e%4 in both operands
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      v8h ph;
#pragma unroll
      for (int e = 0; e < 8; e++) ph[e] = (_Float16)sc[8 * s2 + e];
      const uint4 hw = __builtin_bit_cast(uint4, ph);
      const v8h pl = __builtin_bit_cast(v8h, make_uint4(pa_lo2(sc[8 * s2], sc[8 * s2 + 1], hw.x),
                                                        pa_lo2(sc[8 * s2 + 2], sc[8 * s2 + 3], hw.y),
                                                        pa_lo2(sc[8 * s2 + 4], sc[8 * s2 + 5], hw.z),
                                                        pa_lo2(sc[8 * s2 + 6], sc[8 * s2 + 7], hw.w)));
#pragma unroll
      for (int t = 0; t < HD / 32; t++) {
        const uint16_t *vrow = &s_v[buf][(32 * t + li) * VP + 16 * s2 + 4 * lg];
        const uint2 va = *(const uint2 *)vrow, vb = *(const uint2 *)(vrow + 8);
        const v8h vf = f16x8(make_uint4(va.x, va.y, vb.x, vb.y));
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, ph, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pl, o[t], 0, 0, 0);
      }
    }
    if (kb + 1 < nkb) PA_STORE(buf ^ 1, kb + 1);
  }
#undef PA_LOAD
#undef PA_STORE
#undef PA_RES
  // O^T tile t, register r: dim 32 t + 8 (r/4) + 4 lg + r%4 of query li
  if (SPLIT) {
    if (live) {
      const size_t pr = (size_t)piece * gridDim.z * a.qper + row;
      float *po = a.part_o + pr * a.nq + (size_t)head * HD + 4 * lg;
#pragma unroll
      for (int t = 0; t < HD / 32; t++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
          *(float4 *)(po + 32 * t + 8 * rq) =
              make_float4(o[t][4 * rq], o[t][4 * rq + 1], o[t][4 * rq + 2], o[t][4 * rq + 3]);
      if (lg == 0) *(float2 *)(a.part_ml + (pr * a.heads + head) * 2) = make_float2(m, l);
    }
    return;
  }
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

// The pieces of a split prompt attention merged: per (row, head), M = max
// of the pieces' maxima, L = sum l_p 2^(m_p - M), ctx = sum o_p 2^(m_p - M)
// / L over the pieces that row's query block has; one thread per 4 dims.
__global__ __launch_bounds__(256) void k_prefill_merge(PrefillArgs a, uint32_t hd, uint32_t nrows) {
  const uint32_t per = hd / 4;
  const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (uint64_t)nrows * a.heads * per) return;
  const uint32_t d4 = (uint32_t)(gid % per);
  const uint64_t rh = gid / per;
  const uint32_t head = (uint32_t)(rh % a.heads), row = (uint32_t)(rh / a.heads);
  // the pieces this row's query block was split into (as k_prefill_attn counts them)
  const uint32_t qb = (row % a.qper) / PA_QB;
  const int32_t pos0 = a.pos[0];
  const uint32_t ilast = min(qb * PA_QB + PA_QB - 1, a.qper - 1);
  const int32_t plast = min(pos0 + (int32_t)ilast, (int32_t)a.max_seq - 1);
  const uint32_t nkb_all = plast < 0 ? 0u : (uint32_t)plast / PA_KB + 1;
  const uint32_t np = nkb_all ? (nkb_all + a.kps - 1) / a.kps : 1;
  float mm = -1.0e30f;
  for (uint32_t p = 0; p < np; p++) {
    const float mp = a.part_ml[(((size_t)p * nrows + row) * a.heads + head) * 2];
    mm = mp > mm ? mp : mm;
  }
  float ll = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (uint32_t p = 0; p < np; p++) {
    const size_t pr = (size_t)p * nrows + row;
    const float2 ml = *(const float2 *)(a.part_ml + (pr * a.heads + head) * 2);
    const float sc = nlg_exp2(ml.x - mm);
    ll = fmaf(ml.y, sc, ll);
    const float4 v = *(const float4 *)(a.part_o + pr * a.nq + (size_t)head * hd + 4 * d4);
    acc.x = fmaf(v.x, sc, acc.x);
    acc.y = fmaf(v.y, sc, acc.y);
    acc.z = fmaf(v.z, sc, acc.z);
    acc.w = fmaf(v.w, sc, acc.w);
  }
  const float4 out = ll > 0.0f ? make_float4(acc.x / ll, acc.y / ll, acc.z / ll, acc.w / ll)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  *(float4 *)(a.ctx + (size_t)row * a.nq + (size_t)head * hd + 4 * d4) = out;
}

// The same merge for whole rows (one workgroup per row), then the per-token
// quantisation of k_act_q (amax, gamma = amax / 127, the exact quantiser,
// matrix-core byte order across each quad) straight into the int8 rows the
// output projection's GEMM reads: the merged context never goes to memory.
// Thread t takes float4s t + 256 j of the row; the merge runs in
// k_prefill_merge's operation order and the quantisation in k_act_q's, so
// the int8 rows and gammas are the ones the two launches would leave.
template <int J>
__global__ __launch_bounds__(256) void k_prefill_merge_q(PrefillArgs a, uint32_t hd, uint32_t nrows, uint8_t *xq,
                                                         float *gamma) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x, nf4 = a.nq >> 2, per = hd / 4;
  const uint32_t qb = (row % a.qper) / PA_QB;
  const int32_t pos0 = a.pos[0];
  const uint32_t ilast = min(qb * PA_QB + PA_QB - 1, a.qper - 1);
  const int32_t plast = min(pos0 + (int32_t)ilast, (int32_t)a.max_seq - 1);
  const uint32_t nkb_all = plast < 0 ? 0u : (uint32_t)plast / PA_KB + 1;
  const uint32_t np = nkb_all ? (nkb_all + a.kps - 1) / a.kps : 1;
  float4 v[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const uint32_t f0 = threadIdx.x + 256u * j, f = f0 < nf4 ? f0 : nf4 - 1;
    const uint32_t head = f / per, d4 = f % per;
    float mm = -1.0e30f;
    for (uint32_t p = 0; p < np; p++) {
      const float mp = a.part_ml[(((size_t)p * nrows + row) * a.heads + head) * 2];
      mm = mp > mm ? mp : mm;
    }
    float ll = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t p = 0; p < np; p++) {
      const size_t pr = (size_t)p * nrows + row;
      const float2 ml = *(const float2 *)(a.part_ml + (pr * a.heads + head) * 2);
      const float sc = nlg_exp2(ml.x - mm);
      ll = fmaf(ml.y, sc, ll);
      const float4 x = *(const float4 *)(a.part_o + pr * a.nq + (size_t)head * hd + 4 * d4);
      acc.x = fmaf(x.x, sc, acc.x);
      acc.y = fmaf(x.y, sc, acc.y);
      acc.z = fmaf(x.z, sc, acc.z);
      acc.w = fmaf(x.w, sc, acc.w);
    }
    v[j] = ll > 0.0f && f0 < nf4 ? make_float4(acc.x / ll, acc.y / ll, acc.z / ll, acc.w / ll)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
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
  amax = nlg_block_max_f32<4, true>(amax, red);
  const float g = nlg_gamma_of(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(amax))));
  const float ginv = 1.0f / g;
  const bool fast = quant_fast(g);
  if (threadIdx.x == 0) gamma[row] = g;
  const uint32_t qi = threadIdx.x & 3u;
  const uint32_t sel_lo = 0x0c0c0000u | ((4u + qi) << 8) | qi, sel_hi = 0x00000c0cu | ((4u + qi) << 24) | (qi << 16);
  uint32_t *dst = (uint32_t *)(xq + (size_t)row * a.nq);
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

}  // namespace

int nlg_prefill_attn(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos, uint32_t rows,
                     uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                     float *ctx, hipStream_t st, uint8_t *xq, float *gamma, bool *quantized, uint32_t pos_bound) {
  if (quantized) *quantized = false;
  if (!rows) return NLG_OK;
  if (!q || !kc || !vc || !pos || !ctx) return nlg_fail("prefill attn: null pointer");
  if (head_dim != 64 && head_dim != 128) return nlg_fail("prefill attn: head_dim %u not 64 or 128", head_dim);
  if (!kvheads || heads % kvheads) return nlg_fail("prefill attn: heads %u not a multiple of kv heads %u", heads, kvheads);
  const uint32_t grp = heads / kvheads;
  if (grp != 1 && grp != 2 && grp != 4 && grp != 8) return nlg_fail("prefill attn: heads/kvheads %u not 1, 2, 4 or 8", grp);
  if (!qper || rows % qper) return nlg_fail("prefill attn: rows %u not a multiple of rows per sequence %u", rows, qper);
  if (!max_seq) return nlg_fail("prefill attn: max_seq is 0");
  if ((uint64_t)max_seq * head_dim * 2 >= (1ull << 31))
    return nlg_fail("prefill attn: a cache slot of %u x %u halves exceeds 2 GiB", max_seq, head_dim);
  if (((uintptr_t)q & 15) || ((uintptr_t)kc & 15) || ((uintptr_t)vc & 15) || ((uintptr_t)ctx & 15))
    return nlg_fail("prefill attn: q, caches and ctx must be 16-byte aligned");
  const uint32_t nseq = rows / qper;
  if (nseq > 65535 || kvheads > 65535) return nlg_fail("prefill attn: too many sequences or kv heads");
  PrefillArgs a{q, kc, vc, pos, ctx, qper, heads, kvheads, max_seq, heads * head_dim,
                (1.0f / sqrtf((float)head_dim)) * NLG_LOG2E,  // (/ 1.0 (sqrt (float hd))), in base 2
                nullptr, nullptr, 0, 0};
  const uint32_t nqb = (qper + PA_QB - 1) / PA_QB;
  // Too few workgroups to fill the CUs (one prompt: 16 query blocks x kv
  // heads), and the last query block walks every key block while the first
  // walks one: split each block's keys into pieces of kps key blocks,
  // merged by a second launch.  kps is half the key blocks a prompt
  // starting at position 0 spans (at least 4), so the longest query blocks
  // take two equal pieces (measured at 512 tokens, 20/5 heads: pieces of 8
  // blocks 24.5 us with the merge, of 4 27.2, 6 29.2, 12 28.5, 1 39.8;
  // unsplit 27.2).  The pieces' partials go to a per-stream workspace;
  // without one (a capture that would have to grow it) the launch stays
  // unsplit.
  // Keys reach at most the last prompt position: max_seq, or pos_bound when
  // the caller knows a smaller bound (the stack: the prompt length), which
  // sizes the pieces' workspace by the prompt instead of the cache.
  const uint32_t kreach = pos_bound && pos_bound < max_seq ? pos_bound : max_seq;
  const uint32_t kblocks = (kreach + PA_KB - 1) / PA_KB, kps = nqb / 2 + nqb % 2 > 4 ? nqb / 2 + nqb % 2 : 4;
  if ((uint64_t)nqb * kvheads * nseq < 256 && kblocks > kps) {
    const uint32_t maxp = (kblocks + kps - 1) / kps;
    const size_t o_bytes = (size_t)maxp * rows * a.nq * 4, ml_bytes = (size_t)maxp * rows * heads * 2 * 4;
    uint8_t *ws = (uint8_t *)nlg_scratch_try((o_bytes + 255) / 256 * 256 + ml_bytes, st, 2);
    if (ws && (uint64_t)nqb * maxp <= 0x7fffffffu) {
      a.part_o = (float *)ws;
      a.part_ml = (float *)(ws + (o_bytes + 255) / 256 * 256);
      a.kps = kps;
      a.maxp = maxp;
      const dim3 grid(nqb * maxp, kvheads, nseq), blk(64 * grp);
#define PAS(HD)                                                                              \
  do {                                                                                       \
    if (grp == 1) hipLaunchKernelGGL((k_prefill_attn<HD, 1, true>), grid, blk, 0, st, a);    \
    else if (grp == 2) hipLaunchKernelGGL((k_prefill_attn<HD, 2, true>), grid, blk, 0, st, a); \
    else if (grp == 4) hipLaunchKernelGGL((k_prefill_attn<HD, 4, true>), grid, blk, 0, st, a); \
    else hipLaunchKernelGGL((k_prefill_attn<HD, 8, true>), grid, blk, 0, st, a);             \
  } while (0)
      if (head_dim == 128) PAS(128); else PAS(64);
#undef PAS
      NLG_LAUNCHED("prefill attention (fp16 KV, MFMA, split keys)");
      const uint32_t jq = (a.nq / 4 + 255) / 256;  // float4s per thread of a whole row
      if (xq && gamma && quantized && a.nq % 64 == 0 && jq <= 4) {
        // merged and quantised per row for the output projection
        if (jq <= 1) hipLaunchKernelGGL(k_prefill_merge_q<1>, dim3(rows), dim3(256), 0, st, a, head_dim, rows, xq, gamma);
        else if (jq <= 2) hipLaunchKernelGGL(k_prefill_merge_q<2>, dim3(rows), dim3(256), 0, st, a, head_dim, rows, xq, gamma);
        else if (jq <= 3) hipLaunchKernelGGL(k_prefill_merge_q<3>, dim3(rows), dim3(256), 0, st, a, head_dim, rows, xq, gamma);
        else hipLaunchKernelGGL(k_prefill_merge_q<4>, dim3(rows), dim3(256), 0, st, a, head_dim, rows, xq, gamma);
        NLG_LAUNCHED("prefill attention merge + quantisation");
        *quantized = true;
        return NLG_OK;
      }
      const uint64_t nthr = (uint64_t)rows * heads * (head_dim / 4);
      hipLaunchKernelGGL(k_prefill_merge, dim3((uint32_t)((nthr + 255) / 256)), dim3(256), 0, st, a, head_dim,
                         rows);
      NLG_LAUNCHED("prefill attention merge");
      return NLG_OK;
    }
  }
  const dim3 grid(nqb, kvheads, nseq), blk(64 * grp);
#define PA(HD)                                                                             \
  do {                                                                                     \
    if (grp == 1) hipLaunchKernelGGL((k_prefill_attn<HD, 1, false>), grid, blk, 0, st, a);        \
    else if (grp == 2) hipLaunchKernelGGL((k_prefill_attn<HD, 2, false>), grid, blk, 0, st, a);   \
    else if (grp == 4) hipLaunchKernelGGL((k_prefill_attn<HD, 4, false>), grid, blk, 0, st, a);   \
    else hipLaunchKernelGGL((k_prefill_attn<HD, 8, false>), grid, blk, 0, st, a);                 \
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

// Prompt attention and the attention output projection with its residual,
// as the stack's prefill runs them: when the keys are split (few prompts),
// the pieces are merged and quantised for the projection in one launch
// (k_prefill_merge_q) and the projection's GEMM reads those int8 rows;
// otherwise ctx_ws receives the context and the projection quantises it.
// Both give the bits of nlg_prefill_attn_f16 followed by
// nlg_ternary_linear_residual.
int nlg_prefill_attn_o_resid(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos,
                             uint32_t rows, uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                             uint32_t max_seq, uint32_t pos_bound, float *ctx_ws, const uint32_t *w2,
                             const float *bias, const float *beta, int beta_per_row, const float *res, float *y,
                             uint32_t out, hipStream_t st) {
  const uint32_t nq = heads * head_dim;
  uint8_t *oq = rows >= NLG_BATCHED_MIN && nq % 256 == 0 ? (uint8_t *)nlg_scratch(nlg_batched_scratch_bytes(rows, nq), st)
                                                        : nullptr;
  float *og = oq ? (float *)(oq + ((size_t)rows * nq + 255) / 256 * 256) : nullptr;
  bool quantized = false;
  if (nlg_prefill_attn(q, kc, vc, pos, rows, qper, heads, kvheads, head_dim, max_seq, ctx_ws, st, oq, og, &quantized,
                       pos_bound))
    return NLG_ERR;
  FusedArgs o{};
  o.x = ctx_ws; o.w2 = w2; o.bias = bias; o.beta = beta; o.beta_per_row = beta_per_row; o.seq = rows; o.out = out;
  o.cols = nq; o.y = y; o.ystride = out; o.res = res; o.rstride = out;
  return quantized ? nlg_batched_gemm(o, oq, og, NLG_EPI_RESID, st) : nlg_fused_launch(o, NLG_PRO_NONE, NLG_EPI_RESID, 0, st);
}

extern "C" int nlg_prefill_attn_ternary_linear_residual(const float *q, const uint16_t *kcache,
                                                        const uint16_t *vcache, const int32_t *pos, uint32_t rows,
                                                        uint32_t qper, uint32_t heads, uint32_t kvheads,
                                                        uint32_t head_dim, uint32_t max_seq, float *ctx_ws,
                                                        const uint32_t *w2, const float *bias, const float *beta,
                                                        int beta_per_row, const float *res, float *y, uint32_t out,
                                                        void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!w2 || !beta || !res || !y) return nlg_fail("prefill attn + projection: null pointer");
  return nlg_prefill_attn_o_resid(q, kcache, vcache, pos, rows, qper, heads, kvheads, head_dim, max_seq, 0, ctx_ws,
                                  w2, bias, beta, beta_per_row, res, y, out, nlg_stream(stream));
}
