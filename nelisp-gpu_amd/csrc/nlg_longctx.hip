// nlg_longctx.hip -- the long-context decode attentions, on the reference's
// f32 layouts:
//
//   decode-attn-stream  (kernels.el:404-451)   StreamingLLM: nsink sink slots +
//                       a win-slot ring; K and q rotated in the kernel by their
//                       cache-relative positions (CO/SI tables)
//   attn-stream-entries (kernels.el:1050-1090) the same over an explicit list of
//                       [K/V row base, cache-relative position] pairs
//   decode-attn-paged   (kernels.el:1110-1136) per-sequence attention through a
//                       block table into a shared pool, at the shared POS[0]
//   decode-attn-paged-v (kernels.el:1222-1246) the same at each sequence's LENS[s]
//
// As decode-attn here: a workgroup owns one (sequence, head); its four waves
// take every fourth position; each lane holds rotation pairs (2m, 2m+1) of
// the head dimension (the unit RoPE works on), so a position's q.k product is
// one DPP wave reduction; the waves' running max, sum and context meet in
// LDS.  Scores keep the reference's two passes (max, then sum and context).
// Every access is bounds-checked (reads past a buffer give 0, writes are
// dropped): positions, table entries and entry lists come from device memory.
#include <math.h>

#include "nlg_internal.h"

#define NEG_BIG (-1.0e30f)

namespace {

struct LB {
  const float *p;
  uint32_t n;
};
__device__ __forceinline__ float lld(const LB &b, uint32_t i) { return i < b.n ? b.p[i] : 0.0f; }
__device__ __forceinline__ uint32_t ludiv(uint32_t a, uint32_t b) { return b ? a / b : 0u; }
__device__ __forceinline__ uint32_t lumod(uint32_t a, uint32_t b) { return b ? a % b : 0u; }

enum { LC_STREAM = 0, LC_ENTRIES = 1, LC_PAGED = 2, LC_PAGED_V = 3 };

struct LcArgs {
  LB q, ck, cv, aux, table, co, si;  // aux: POS, ENT or LENS
  float *c;
  uint32_t nc;
  uint32_t dim, heads, kvheads, hd, grp, kvdim, half, hslots, domain;
  uint32_t nsink, win;  // stream
  uint32_t ne, qcrel;   // entries
  uint32_t bs, mbps;    // paged
  uint32_t tabn;        // table entries readable (paged)
};

// Position r's K/V row base (the head's first element) and, for the RoPE
// modes, its cache-relative position.
template <int MODE>
__device__ __forceinline__ uint32_t lc_row(const LcArgs &a, uint32_t bb, uint32_t kvh, uint32_t r, uint32_t woff,
                                           uint32_t &crel) {
  if (MODE == LC_STREAM) {
    uint32_t slot = r;
    if (r >= a.nsink) slot = a.nsink + lumod(woff + (r - a.nsink), a.win);
    crel = r;
    return slot * a.kvdim + kvh * a.hd;
  } else if (MODE == LC_ENTRIES) {
    const uint32_t base = nlg_f2u(lld(a.aux, 2 * r));
    crel = nlg_f2u(lld(a.aux, 2 * r + 1));
    return base + kvh * a.hd;
  } else {
    const uint32_t lb = ludiv(r, a.bs), off = lumod(r, a.bs);
    const uint32_t phys = nlg_f2u(lld(a.table, bb * a.mbps + lb));
    crel = 0;
    return (phys * a.bs + off) * a.kvdim + kvh * a.hd;
  }
}

// EPP: rotation pairs per lane (hd <= 128 EPP).
template <int MODE, int EPP>
__global__ __launch_bounds__(256) void k_lc_attn(LcArgs a) {
  constexpr bool ROPE = MODE == LC_STREAM || MODE == LC_ENTRIES;
  __shared__ float s_ctx[4][128 * EPP];
  __shared__ float s_z[4], s_mx[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t bb = blockIdx.x / a.hslots, h = blockIdx.x % a.hslots;
  const uint32_t kvh = ludiv(h, a.grp);
  const uint32_t c0q = bb * a.dim + h * a.hd;
  const float coef = 1.0f / sqrtf((float)a.hd);
  // positions attended, the stream's ring offset and the query's position
  uint32_t len = 0, woff = 0, qcrel = 0;
  if (MODE == LC_STREAM) {
    const uint32_t pos = nlg_f2u(lld(a.aux, 0)), cap = a.nsink + a.win;
    len = pos + 1;
    if (len > cap) len = cap;
    uint32_t start = a.nsink;
    if (pos >= cap) start = (pos - a.win) + 1;
    woff = lumod(start - a.nsink, a.win);
    qcrel = pos;
    if (qcrel >= cap) qcrel = cap - 1;
  } else if (MODE == LC_ENTRIES) {
    len = a.ne;
    qcrel = a.qcrel;
  } else {
    len = nlg_f2u(lld(a.aux, MODE == LC_PAGED_V ? bb : 0u)) + 1;
  }
  // Paged positions whose table slot lies past the TABLE buffer are not
  // walked: they count as all-zero rows (score 0, zero V), so a wild position
  // cannot make the loop run for billions of trips.
  uint32_t jl = len;
  if (MODE == LC_PAGED || MODE == LC_PAGED_V) {
    const uint64_t first = (uint64_t)bb * a.mbps;
    const uint64_t ext = first < a.tabn ? (uint64_t)(a.tabn - first) * a.bs : 0;
    if ((uint64_t)jl > ext) jl = (uint32_t)ext;
  }
  // q (rotated by the query's position in the RoPE modes)
  float q0[EPP], q1[EPP];
#pragma unroll
  for (int e = 0; e < EPP; e++) {
    const uint32_t m = lane + 64 * e, t0 = 2 * m;
    const float x0 = t0 < a.hd ? lld(a.q, c0q + t0) : 0.0f;
    const float x1 = t0 + 1 < a.hd ? lld(a.q, c0q + t0 + 1) : 0.0f;
    if (ROPE && m < a.half) {
      const uint32_t qi = qcrel * a.half + m;
      const float qc = lld(a.co, qi), qs = lld(a.si, qi);
      q0[e] = __fsub_rn(__fmul_rn(x0, qc), __fmul_rn(x1, qs));
      q1[e] = __fadd_rn(__fmul_rn(x0, qs), __fmul_rn(x1, qc));
    } else {
      q0[e] = x0;
      q1[e] = x1;
    }
  }
  auto score = [&](uint32_t kb, uint32_t crel) {
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < EPP; e++) {
      const uint32_t m = lane + 64 * e, t0 = 2 * m;
      const float k0 = t0 < a.hd ? lld(a.ck, kb + t0) : 0.0f;
      const float k1 = t0 + 1 < a.hd ? lld(a.ck, kb + t0 + 1) : 0.0f;
      if (ROPE) {
        const uint32_t ci = crel * a.half + m;
        const float cc = lld(a.co, ci), ss = lld(a.si, ci);
        const float kr0 = __fsub_rn(__fmul_rn(k0, cc), __fmul_rn(k1, ss));
        const float kr1 = __fadd_rn(__fmul_rn(k0, ss), __fmul_rn(k1, cc));
        if (m < a.half) d = __fadd_rn(d, __fadd_rn(__fmul_rn(q0[e], kr0), __fmul_rn(q1[e], kr1)));
      } else {
        d = __fadd_rn(d, __fadd_rn(__fmul_rn(q0[e], k0), __fmul_rn(q1[e], k1)));
      }
    }
    return __fmul_rn(nlg_wave_sum_f32(d), coef);
  };
  // pass 1: the maximum score (seeded -1e30 as the reference)
  float mx = NEG_BIG;
  for (uint32_t r = w; r < jl; r += 4) {
    uint32_t crel;
    const uint32_t kb = lc_row<MODE>(a, bb, kvh, r, woff, crel);
    const float s = score(kb, crel);
    if (s > mx) mx = s;
  }
  if (jl < len && 0.0f > mx) mx = 0.0f;
  if (lane == 0) s_mx[w] = mx;
  __syncthreads();
  mx = s_mx[0];
  for (int i = 1; i < 4; i++) mx = s_mx[i] > mx ? s_mx[i] : mx;
  // pass 2: z and ctx
  float z = 0.0f, cx0[EPP], cx1[EPP];
#pragma unroll
  for (int e = 0; e < EPP; e++) cx0[e] = cx1[e] = 0.0f;
  for (uint32_t r = w; r < jl; r += 4) {
    uint32_t crel;
    const uint32_t kb = lc_row<MODE>(a, bb, kvh, r, woff, crel);
    const float ee = expf(__fsub_rn(score(kb, crel), mx));
    z = __fadd_rn(z, ee);
#pragma unroll
    for (int e = 0; e < EPP; e++) {
      const uint32_t t0 = 2 * (lane + 64 * e);
      if (t0 < a.hd) cx0[e] = __fadd_rn(cx0[e], __fmul_rn(ee, lld(a.cv, kb + t0)));
      if (t0 + 1 < a.hd) cx1[e] = __fadd_rn(cx1[e], __fmul_rn(ee, lld(a.cv, kb + t0 + 1)));
    }
  }
#pragma unroll
  for (int e = 0; e < EPP; e++) {
    const uint32_t t0 = 2 * (lane + 64 * e);
    s_ctx[w][t0] = cx0[e];
    s_ctx[w][t0 + 1] = cx1[e];
  }
  if (lane == 0) s_z[w] = z;
  __syncthreads();
  if (w == 0) {
    float zt = __fadd_rn(__fadd_rn(s_z[0], s_z[1]), __fadd_rn(s_z[2], s_z[3]));
    if (jl < len) zt = __fadd_rn(zt, __fmul_rn((float)(len - jl), expf(__fsub_rn(0.0f, mx))));
#pragma unroll
    for (int e = 0; e < 2 * EPP; e++) {
      const uint32_t t = lane + 64 * e;
      const float ct = __fadd_rn(__fadd_rn(s_ctx[0][t], s_ctx[1][t]), __fadd_rn(s_ctx[2][t], s_ctx[3][t]));
      const uint32_t oc = h * a.hd + t, idx = bb * a.dim + oc;
      if (t < a.hd && oc < a.dim && idx < a.domain && idx < a.nc) a.c[idx] = ct / zt;
    }
  }
}

template <int MODE>
int lc_launch(LcArgs &a, uint32_t B, uint32_t groups, hipStream_t st, const char *k) {
  if (!a.heads || !a.kvheads) return nlg_fail("%s: heads and kvheads must be nonzero", k);
  a.hd = a.dim / a.heads;
  a.grp = a.heads / a.kvheads;
  a.kvdim = a.kvheads * a.hd;
  a.half = a.hd / 2;
  if (!a.hd) return NLG_OK;
  if (a.hd > 512) return nlg_fail("%s: head dim %u > 512", k, a.hd);
  a.hslots = (a.dim + a.hd - 1) / a.hd;
  const uint64_t dom = nlg_domain((uint64_t)B * a.dim, groups);
  if (!dom) return NLG_OK;
  a.domain = (uint32_t)dom;
  const uint32_t seqs = (uint32_t)((dom + a.dim - 1) / a.dim);
  const dim3 g(seqs * a.hslots), blk(256);
  if (a.hd <= 128) hipLaunchKernelGGL((k_lc_attn<MODE, 1>), g, blk, 0, st, a);
  else if (a.hd <= 256) hipLaunchKernelGGL((k_lc_attn<MODE, 2>), g, blk, 0, st, a);
  else hipLaunchKernelGGL((k_lc_attn<MODE, 4>), g, blk, 0, st, a);
  NLG_LAUNCHED(k);
  return NLG_OK;
}

LB lb_of(const nlg_buffer &b) { return LB{(const float *)b.ptr, b.nfloats}; }

}  // namespace

// decode-attn-stream: Q CK CV POS CO SI C; push (dim heads kvheads nsink win)
int L_decode_attn_stream(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  LcArgs a{};
  a.q = lb_of(b[0]); a.ck = lb_of(b[1]); a.cv = lb_of(b[2]); a.aux = lb_of(b[3]);
  a.co = lb_of(b[4]); a.si = lb_of(b[5]); a.c = (float *)b[6].ptr; a.nc = b[6].nfloats;
  a.dim = p[0]; a.heads = p[1]; a.kvheads = p[2]; a.nsink = p[3]; a.win = p[4];
  // the loop runs over at most nsink + win entries: the caches must hold them
  if (a.heads && a.kvheads) {
    const uint64_t cap = (uint32_t)(a.nsink + a.win), kvdim = (uint64_t)a.kvheads * (a.dim / a.heads);
    const uint64_t lim = b[1].nfloats > b[2].nfloats ? b[1].nfloats : b[2].nfloats;
    if (cap * kvdim > lim)
      return nlg_fail("decode-attn-stream: caches hold %llu floats, nsink+win = %llu entries need %llu",
                      (unsigned long long)lim, (unsigned long long)cap, (unsigned long long)(cap * kvdim));
  }
  return lc_launch<LC_STREAM>(a, 1, groups, st, "decode-attn-stream");
}

// attn-stream-entries: Q CK CV ENT CO SI C; push (dim heads kvheads ne qcrel)
int L_attn_stream_entries(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  LcArgs a{};
  a.q = lb_of(b[0]); a.ck = lb_of(b[1]); a.cv = lb_of(b[2]); a.aux = lb_of(b[3]);
  a.co = lb_of(b[4]); a.si = lb_of(b[5]); a.c = (float *)b[6].ptr; a.nc = b[6].nfloats;
  a.dim = p[0]; a.heads = p[1]; a.kvheads = p[2]; a.ne = p[3]; a.qcrel = p[4];
  if (nlg_need(b, 3, 2ull * a.ne, "attn-stream-entries")) return NLG_ERR;
  return lc_launch<LC_ENTRIES>(a, 1, groups, st, "attn-stream-entries");
}

// decode-attn-paged(-v): Q CK CV POS|LENS TABLE C; push (B dim heads kvheads bs mbps)
static int paged(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st, bool per_seq) {
  LcArgs a{};
  a.q = lb_of(b[0]); a.ck = lb_of(b[1]); a.cv = lb_of(b[2]); a.aux = lb_of(b[3]);
  a.table = lb_of(b[4]); a.tabn = b[4].nfloats; a.c = (float *)b[5].ptr; a.nc = b[5].nfloats;
  a.dim = p[1]; a.heads = p[2]; a.kvheads = p[3]; a.bs = p[4]; a.mbps = p[5];
  if (per_seq) return lc_launch<LC_PAGED_V>(a, p[0], groups, st, "decode-attn-paged-v");
  return lc_launch<LC_PAGED>(a, p[0], groups, st, "decode-attn-paged");
}
int L_decode_attn_paged(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return paged(b, p, groups, st, false);
}
int L_decode_attn_paged_v(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {
  return paged(b, p, groups, st, true);
}
