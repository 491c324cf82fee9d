// nlg_dattn.hip -- fp16 KV-cache decode attention.
//
// k_attn_part + k_attn_merge: single-query GQA attention over fp16 KV
// caches (decode-attn(-b), kernels.el:315-338, :366-390: scale 1/sqrt(hd),
// max seeded at -1e30, C = sum(e*V)/sum(e)), split over chunks of positions.
// Each workgroup of the first pass handles one (chunk, kv head, sequence)
// for all the query heads of that kv head, so K and V are read from HBM once;
// a second launch merges the chunks (max-rescaled sums).  The same chunk pass
// serves contiguous caches [seq][kvheads][max_seq][hd], paged pools
// (decode-attn-paged-v, kernels.el:1222-1246) through a block table, and
// StreamingLLM ring caches (decode-attn-stream, kernels.el:409-451): nsink
// sink slots + a win-slot ring, keys and the query rotated by their
// cache-relative positions.
#include <math.h>

#include "nlg_internal.h"

// fp16 element e (0..7) of eight packed in a uint4, as f32 (exact)
__device__ __forceinline__ float f16x8_at(const uint4 &u, int e) {
  const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
  return (float)__builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu)));
}

// -------------------------------------------------- fp16 decode attention

struct AttnArgs {
  const float *q;           // [B x heads*hd]
  const uint16_t *kc, *vc;  // [B][kvheads][max_seq][hd] fp16 bits
  const int32_t *pos;       // attend positions 0..pos[0]
  float *pctx;              // [B][nchunk][heads*hd]: sum of e*V over the chunk
  float *pmz;               // [B][nchunk][heads][2]: chunk max, sum of e
  uint32_t heads, kvheads, max_seq, nchunk;
  uint32_t qper;            // 0: row z = sequence z at pos[0]; else sequence z/qper at pos[0] + z%qper
  uint32_t grp;             // query heads per kv head (a workgroup takes G <= grp of them)
  float coef;               // log2(e)/sqrt(hd): scores in base 2
  // paged caches (PG): pools [block][bs][kvheads][hd]; sequence b's position p
  // lives in block table[b*mbps + p/bs] at offset p%bs; its own position is
  // lens[b] (or pos[0] when lens is null); blocks >= npool read as zeros
  const int32_t *table, *lens;
  uint32_t bs, mbps, npool;
  // ring caches (AM_RING): [B][kvheads][nsink + win][hd], sequence b at
  // stream position pos[b]; co/si: [>= nsink + win][hd/2] rotation tables
  const float *co, *si;
  uint32_t nsink, win;
  // entry lists (AM_ENTRIES): sequence b attends ent[b][0..max_seq) = (slot,
  // rank) int32 pairs over its cache [kvheads][nslots][hd]; the query's rank
  // is lens[b]; slots outside [0, nslots) read as zero rows, ranks outside
  // [0, trows) as zero rotations
  const int32_t *ent;
  uint32_t nslots, trows;
  // one query head per workgroup (G == 1): units (row, kv head, chunk) on a
  // 1-D grid, the grp workgroups of a unit on one XCD (see attn_unit)
  uint32_t nunits;
};

// how k_attn_part finds position p's K/V row; AM_NT added to a mode: K and V
// read with non-temporal loads
enum { AM_CONTIG = 0, AM_PAGED = 1, AM_RING = 2, AM_ENTRIES = 3, AM_NT = 8 };

// K/V row loads, plain or non-temporal
template <bool NT>
__device__ __forceinline__ uint4 kv_ld(const uint16_t *p) {
  return NT ? nlg_ld_stream((const uint4 *)p) : *(const uint4 *)p;
}

// A launch that attends this many bytes of K and V streams them with
// non-temporal loads: a decode step's layers then need more than the 256 MB
// MALL, which cannot keep them from one step to the next anyway (measured at
// the config-5 shape: B=32, 63 MB per layer, 13.9k -> 14.4k tok/s), while
// smaller caches (B=1: 2 MB per layer) are left to be served from it.
#define ATTN_NT_BYTES (16ull << 20)

__device__ __forceinline__ float f4_at(const float4 &v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// Sum over aligned groups of L lanes (L = 8 or 16); every lane gets its
// group's sum.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  v = v + __int_as_float(nlg_dpp<0xB1>(__float_as_int(v)));   // quad_perm [1,0,3,2]
  v = v + __int_as_float(nlg_dpp<0x4E>(__float_as_int(v)));   // quad_perm [2,3,0,1]
  v = v + __int_as_float(nlg_dpp<0x141>(__float_as_int(v)));  // row_half_mirror
  if (L == 16) v = v + __int_as_float(nlg_dpp<0x140>(__float_as_int(v)));  // row_mirror
  return v;
}

// Positions per workgroup for head dim HD: 8 waves x NI instructions x
// (64 / (HD/8)) positions per instruction; NI = 8 when 4 would need more
// chunks than the O-projection's prologue merges.
#define ATTN_WAVES 8
static inline uint32_t attn_ni(uint32_t hd, uint32_t max_seq) {
  const uint32_t cs4 = ATTN_WAVES * 4u * (64u / (hd / 8u));
  return (max_seq + cs4 - 1) / cs4 > NLG_ATTN_MAX_CHUNKS ? 8u : 4u;
}
static inline uint32_t attn_chunks(uint32_t hd, uint32_t max_seq) {
  const uint32_t cs = ATTN_WAVES * attn_ni(hd, max_seq) * (64u / (hd / 8u));
  return (max_seq + cs - 1) / cs;
}
uint32_t nlg_attn_chunk_count(uint32_t head_dim, uint32_t max_seq) { return attn_chunks(head_dim, max_seq); }

// Pass 1: one workgroup per (chunk, kv head, sequence) scores its chunk's
// positions for every query head of that kv head (K and V read once) and
// stores the chunk's max m, sum z = sum(exp(s - m)) and sum(exp(s - m) * V).
// Lanes hold 8 dimensions of one position: LPP = HD/8 lanes per position,
// PPI = 64/LPP positions per wave instruction.  Every K and V load of the
// workgroup is issued before the first score is computed.
//
// In a ring cache (AM_RING) chunk positions are cache-relative ranks r:
// rank r < nsink is sink slot r, later ranks walk the ring from its oldest
// entry; K is rotated by r and q by the query's rank (CO/SI tables, pairs
// (2m, 2m+1)) before the product, as decode-attn-stream does.  An entry
// list (AM_ENTRIES, attn-stream-entries) names each attended row's slot and
// rank explicitly; chunk positions index the list.
// v if ok, else zeros: per component, so that no select of whole vectors
// is lowered through private memory
__device__ __forceinline__ uint4 keep_u4(bool ok, uint4 v) {
  return make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);
}
__device__ __forceinline__ float4 keep_f4(bool ok, float4 v) {
  return make_float4(ok ? v.x : 0.0f, ok ? v.y : 0.0f, ok ? v.z : 0.0f, ok ? v.w : 0.0f);
}

template <int HD, int G, int NI, int MODE>
__global__ __launch_bounds__(512) void k_attn_part(AttnArgs a) {
  constexpr int BM = MODE & ~AM_NT;
  constexpr bool NT = (MODE & AM_NT) != 0;
  constexpr bool PG = BM == AM_PAGED, RG = BM == AM_RING || BM == AM_ENTRIES, EN = BM == AM_ENTRIES;
  constexpr int LPP = HD / 8, PPI = 64 / LPP, PW = NI * PPI, NW = ATTN_WAVES, CS = NW * PW;
  __shared__ float s_m[NW][G], s_z[NW][G];
  __shared__ float s_ctx[NW][G][HD];
  asm volatile("" ::"s"(a.q), "s"(a.kc), "s"(a.vc), "s"(a.pos), "s"(a.pctx), "s"(a.pmz), "s"(a.heads),
               "s"(a.kvheads), "s"(a.max_seq), "s"(a.nchunk), "s"(a.coef));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // workgroup: chunk c, query heads h0 .. h0+G-1 (all of one kv head), query row qr
  uint32_t c, h0, qr;
  if (G == 1) {
    // Workgroups are dealt to the 8 XCDs round-robin by id, and each XCD
    // has its own L2: the grp query heads of one (row, kv head, chunk) unit
    // get ids u%8 + 8(q + grp*(u/8)), all on XCD u%8, so the unit's K/V rows
    // come from HBM once and from that L2 for the other heads.
    const uint32_t id = blockIdx.x, rest = id >> 3, q = rest % a.grp, u = (id & 7u) + 8u * (rest / a.grp);
    if (u >= a.nunits) return;
    c = u % a.nchunk;
    const uint32_t r2 = u / a.nchunk;
    h0 = (r2 % a.kvheads) * a.grp + q;
    qr = r2 / a.kvheads;
  } else {
    c = blockIdx.x; h0 = blockIdx.y * G; qr = blockIdx.z;
  }
  const uint32_t kvh = h0 / a.grp;
  const uint32_t b = a.qper ? qr / a.qper : qr;                         // its sequence
  const size_t cb = (size_t)qr * a.nchunk + c;
  float *pctx = a.pctx + cb * a.heads * HD + (size_t)h0 * HD;
  float *pmz = a.pmz + (cb * a.heads + h0) * 2;
  const uint32_t p0 = c * CS;
  // For small caches K, V and q are fetched before the position arrives
  // (addresses clamped to the cache, not to the position), so the position's
  // fetch is not a round trip ahead of theirs; positions past it are masked
  // afterwards.
  const int d0 = 8 * (lane % LPP), grp = lane / LPP;
  const size_t slot = (size_t)b * a.kvheads + kvh;
  const uint16_t *kb = a.kc + slot * a.max_seq * HD + d0;
  const uint16_t *vb = a.vc + slot * a.max_seq * HD + d0;
  // q first: loads retire in issue order, so the first score then waits
  // only for its own K row, and the scores overlap the rest of the stream
  const float *qb = a.q + (size_t)qr * a.heads * HD + (size_t)h0 * HD + d0;
  float q[G][8];
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float4 q0 = *(const float4 *)(qb + h * HD), q1 = *(const float4 *)(qb + h * HD + 4);
    q[h][0] = q0.x; q[h][1] = q0.y; q[h][2] = q0.z; q[h][3] = q0.w;
    q[h][4] = q1.x; q[h][5] = q1.y; q[h][6] = q1.z; q[h][7] = q1.w;
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 kr[NI], vr[NI];
  float4 rc[NI], rs[NI];  // ring: the ranks' rotation pairs (cos, sin)
  uint32_t pp[NI];
  uint32_t len = 0, qrank = 0;
  // paged / entries: bit i set when row i is a real cache row (else it reads
  // as zeros) and, for entries, when its rotation is real (else zero).  The
  // zeros are applied where a row is used, not where it is loaded: a select
  // on a row in flight waits for it, and one after each load put the rows'
  // fetches one behind the other.
  uint32_t rowm = 0, rotm = 0;
  // Rows fetched: positions clamp to lim - 1.  Large caches (NT) read the
  // position first so that rows past it are never fetched (their addresses
  // clamp to the last attended row, a cache hit): bytes over latency.  Small
  // ones fetch the whole chunk while the position is in flight.
  uint32_t lim = a.max_seq;
  if (NT && !RG) {
    const int32_t pr = PG ? (a.lens ? a.lens[b] : a.pos[0]) : a.pos[0] + (a.qper ? (int32_t)(qr % a.qper) : 0);
    lim = (pr < 0 ? 0u : ((uint32_t)pr >= a.max_seq ? a.max_seq - 1 : (uint32_t)pr)) + 1;
  }
  if (EN) {
    // the list entries first, then the rows and rotations they name
    const int2 *eb = (const int2 *)(a.ent + (size_t)b * a.max_seq * 2);
    const uint16_t *kbe = a.kc + slot * a.nslots * HD + d0, *vbe = a.vc + slot * a.nslots * HD + d0;
    int2 ev[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      pp[i] = p0 + w * PW + i * PPI + grp;
      ev[i] = eb[pp[i] < a.max_seq ? pp[i] : a.max_seq - 1];
    }
    __builtin_amdgcn_sched_barrier(0);  // all entries in flight before the first use
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const bool sok = ev[i].x >= 0 && (uint32_t)ev[i].x < a.nslots;
      const bool rok = ev[i].y >= 0 && (uint32_t)ev[i].y < a.trows;
      const size_t sl = sok ? (uint32_t)ev[i].x : 0u, rk = rok ? (uint32_t)ev[i].y : 0u;
      kr[i] = kv_ld<NT>(kbe + sl * HD);
      vr[i] = kv_ld<NT>(vbe + sl * HD);
      rc[i] = *(const float4 *)(a.co + rk * (HD / 2) + d0 / 2);
      rs[i] = *(const float4 *)(a.si + rk * (HD / 2) + d0 / 2);
      rowm |= sok ? 1u << i : 0u;
      rotm |= rok ? 1u << i : 0u;
    }
    __builtin_amdgcn_sched_barrier(0);
    len = a.max_seq;
    const int32_t qk = a.lens[b];
    qrank = qk >= 0 && (uint32_t)qk < a.trows ? (uint32_t)qk : a.trows;  // trows: a zero rotation
  } else if (RG) {
    // the stream position first: it fixes the ring's oldest slot
    const int32_t ps = a.pos[b];
    const uint32_t pos = ps < 0 ? 0u : (uint32_t)ps, cap = a.max_seq;
    len = pos + 1 < cap ? pos + 1 : cap;  // pos + 1 > 0: pos < 2^31
    const uint32_t start = pos >= cap ? pos - a.win + 1 : a.nsink;
    const uint32_t woff = (start - a.nsink) % a.win;
    qrank = pos < cap ? pos : cap - 1;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      pp[i] = p0 + w * PW + i * PPI + grp;
      const uint32_t pc = pp[i] < cap ? pp[i] : cap - 1;
      uint32_t sl = pc;
      if (pc >= a.nsink) {
        const uint32_t t = woff + (pc - a.nsink);  // < 2 win
        sl = a.nsink + (t >= a.win ? t - a.win : t);
      }
      kr[i] = kv_ld<NT>(kb + (size_t)sl * HD);
      vr[i] = kv_ld<NT>(vb + (size_t)sl * HD);
      rc[i] = *(const float4 *)(a.co + (size_t)pc * (HD / 2) + d0 / 2);
      rs[i] = *(const float4 *)(a.si + (size_t)pc * (HD / 2) + d0 / 2);
    }
  } else if (PG) {
    // the block-table entry first, then K and V of that block's row
    const int32_t *trow = a.table + (size_t)b * a.mbps;
    int32_t ph[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      pp[i] = p0 + w * PW + i * PPI + grp;
      const uint32_t pc = pp[i] < lim ? pp[i] : lim - 1;
      ph[i] = trow[pc / a.bs];
    }
    // all table entries in flight before the first use: left to itself the
    // scheduler issued each entry's load after the previous row's address
    // (one full memory round trip per position)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const uint32_t pc = pp[i] < lim ? pp[i] : lim - 1;
      const bool ok = ph[i] >= 0 && (uint32_t)ph[i] < a.npool;
      const size_t row = (((size_t)(ok ? ph[i] : 0) * a.bs + pc % a.bs) * a.kvheads + kvh) * HD + d0;
      kr[i] = kv_ld<NT>(a.kc + row);
      vr[i] = kv_ld<NT>(a.vc + row);
      rowm |= ok ? 1u << i : 0u;
    }
    __builtin_amdgcn_sched_barrier(0);
  } else {
#pragma unroll
    for (int i = 0; i < NI; i++) {
      pp[i] = p0 + w * PW + i * PPI + grp;
      const uint32_t pc = pp[i] < lim ? pp[i] : lim - 1;
      kr[i] = kv_ld<NT>(kb + (size_t)pc * HD);
      vr[i] = kv_ld<NT>(vb + (size_t)pc * HD);
    }
  }
  if (RG) {  // q rotated by the query's rank
    const bool qok = !EN || qrank < a.trows;
    const size_t qo = (size_t)(qok ? qrank : 0u) * (HD / 2) + d0 / 2;
    const float4 f0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 qc = qok ? *(const float4 *)(a.co + qo) : f0;
    const float4 qs = qok ? *(const float4 *)(a.si + qo) : f0;
#pragma unroll
    for (int h = 0; h < G; h++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float x0 = q[h][2 * j], x1 = q[h][2 * j + 1], c = f4_at(qc, j), sn = f4_at(qs, j);
        q[h][2 * j] = x0 * c - x1 * sn;
        q[h][2 * j + 1] = x0 * sn + x1 * c;
      }
    }
  } else {
    const int32_t pr = PG ? (a.lens ? a.lens[b] : a.pos[0]) : a.pos[0] + (a.qper ? (int32_t)(qr % a.qper) : 0);
    len = (pr < 0 ? 0u : ((uint32_t)pr >= a.max_seq ? a.max_seq - 1 : (uint32_t)pr)) + 1;
  }
  if (p0 >= len) {  // block-uniform: a chunk past the position adds nothing
    for (int i = threadIdx.x; i < G * HD; i += NW * 64) pctx[i] = 0.0f;
    if (threadIdx.x < G) {
      pmz[2 * threadIdx.x] = -1.0e30f;
      pmz[2 * threadIdx.x + 1] = 0.0f;
    }
    return;
  }
  float s[NI][G];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    float kf[8];
    const uint4 ki = PG || EN ? keep_u4((rowm >> i) & 1u, kr[i]) : kr[i];
#pragma unroll
    for (int j = 0; j < 8; j++) kf[j] = f16x8_at(ki, j);
    if (RG) {  // K rotated by its rank
      const bool rk = !EN || ((rotm >> i) & 1u);
      const float4 ci = keep_f4(rk, rc[i]), si = keep_f4(rk, rs[i]);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float k0 = kf[2 * j], k1 = kf[2 * j + 1], c = f4_at(ci, j), sn = f4_at(si, j);
        kf[2 * j] = k0 * c - k1 * sn;
        kf[2 * j + 1] = k0 * sn + k1 * c;
      }
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; j++) d = fmaf(q[h][j], kf[j], d);
      d = group_sum<LPP>(d);
      s[i][h] = pp[i] < len ? d * a.coef : -INFINITY;  // (q.k / sqrt(hd)) * log2(e)
    }
  }
  float m[G], z[G], ctx[G][8];
#pragma unroll
  for (int h = 0; h < G; h++) {
    float mm = -1.0e30f;
#pragma unroll
    for (int i = 0; i < NI; i++) mm = s[i][h] > mm ? s[i][h] : mm;
    for (int off = LPP; off < 64; off <<= 1) {
      const float o = __shfl_xor(mm, off);
      mm = o > mm ? o : mm;
    }
    m[h] = mm;
    z[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) ctx[h][j] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < NI; i++) {
    // rows past the position are zeros here, as rows outside a pool are: the
    // score's -inf makes e 0, but a cache row nobody wrote may hold NaN or
    // Inf bits, and 0 x NaN is NaN
    const uint4 vi = keep_u4(EN ? (rowm >> i) & 1u : (pp[i] < len && (!PG || ((rowm >> i) & 1u))), vr[i]);
#pragma unroll
    for (int h = 0; h < G; h++) {
      const float e = nlg_exp2(s[i][h] - m[h]);
      z[h] = z[h] + e;
#pragma unroll
      for (int j = 0; j < 8; j++) ctx[h][j] = fmaf(e, f16x8_at(vi, j), ctx[h][j]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    for (int off = LPP; off < 64; off <<= 1) {
      z[h] = z[h] + __shfl_xor(z[h], off);
#pragma unroll
      for (int j = 0; j < 8; j++) ctx[h][j] = ctx[h][j] + __shfl_xor(ctx[h][j], off);
    }
    if (grp == 0) {
#pragma unroll
      for (int j = 0; j < 8; j++) s_ctx[w][h][d0 + j] = ctx[h][j];
    }
    if (lane == 0) {
      s_m[w][h] = m[h];
      s_z[w][h] = z[h];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * HD; idx += NW * 64) {
    const int h = idx / HD, d = idx % HD;
    float mm = s_m[0][h];
#pragma unroll
    for (int k = 1; k < NW; k++) mm = s_m[k][h] > mm ? s_m[k][h] : mm;
    float zz = 0.0f, cx = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; k++) {
      const float sc = nlg_exp2(s_m[k][h] - mm);
      zz = fmaf(s_z[k][h], sc, zz);
      cx = fmaf(s_ctx[k][h][d], sc, cx);
    }
    pctx[idx] = cx;
    if (d == 0) {
      pmz[2 * h] = mm;
      pmz[2 * h + 1] = zz;
    }
  }
}

// The chunk pass on the matrix cores, for head_dim 128, 4 query heads per
// kv head and 256-position chunks over contiguous caches: the same
// workgroups, chunks and outputs as k_attn_part<128, 4, 8, MODE>, over
// contiguous caches or (RG) StreamingLLM ring caches (chunk positions are
// cache-relative ranks; each K row is rotated by its rank in f32 and, like
// q, split into fp16 hi + lo, three products per step: hi.hi, lo.hi, hi.lo).  Wave w
// takes positions p0 + 32 w .. + 31 of its chunk for the 4 query heads, on
// v_mfma_f32_16x16x32_f16 (layout, checked on gfx950: lane 16g + i holds
// A[i][8g..8g+7] and B[8g..8g+7][i]; result r of lane l is C[4(l/16) + r][l % 16]):
//  * S^T = K Q^T per 16-position block b: A = K (lane (g, i): position
//    16b + i, dims 32s + 8g.. at step s), B = q as fp16 hi + lo halves
//    (columns 0..3 the heads, the rest zero), so lane (g, j < 4) receives
//    head j's scores of positions 16b + 4g + r.
//  * Those 8 values of a lane are exactly what the B operand P^T of
//    O^T = V^T P^T needs (k slot 8g + 4b + r <-> position 16b + 4g + r), as
//    fp16 hi + lo halves: no exchange between lanes.
//  * V^T in that slot order comes from a per-wave LDS tile: each lane loads
//    4 consecutive positions x 8 dims (every load instruction reads 4 whole
//    rows) and writes each dim's 4 values as one 8-byte run of its V^T row;
//    lane (g, i) then reads its A operand (dim 16n + i, slots 8g..8g+7).
// Scores and probabilities carry ~22 bits through the hi + lo halves; the
// matrix cores sum in their own order.  The wave's (max, sum, context)
// merge across the 8 waves as in k_attn_part (each wave's context goes to
// its own V^T tile once the tile is read).  A VALU-only copy of the pass
// spent most of its time on the ~1,100 instructions per wave of the dots,
// reductions and conversions; here they are 32 matrix-core steps per wave.
#define AMF_PITCH 36  // V^T tile row pitch in 16-bit elements (32 slots + 4: 8-byte aligned rows)

template <bool NT, bool RG>
__global__ __launch_bounds__(512, 4) void k_attn_mfma(AttnArgs a) {
  constexpr int HD = 128, G = 4, NW = ATTN_WAVES, PW = 32, CS = NW * PW;
  typedef _Float16 v8h __attribute__((ext_vector_type(8)));
  typedef float v4f __attribute__((ext_vector_type(4)));
  __shared__ float s_m[NW][G], s_z[NW][G];
  // per wave: its V^T tile, then its context [G][HD] (f32)
  __shared__ __align__(16) uint16_t s_vt[NW][HD * AMF_PITCH];
  asm volatile("" ::"s"(a.q), "s"(a.kc), "s"(a.vc), "s"(a.pos), "s"(a.pctx), "s"(a.pmz), "s"(a.heads),
               "s"(a.kvheads), "s"(a.max_seq), "s"(a.nchunk), "s"(a.coef));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const uint32_t c = blockIdx.x, h0 = blockIdx.y * G, qr = blockIdx.z;
  const uint32_t kvh = h0 / a.grp;
  const uint32_t b = a.qper ? qr / a.qper : qr;  // its sequence
  const size_t cb = (size_t)qr * a.nchunk + c;
  float *pctx = a.pctx + cb * a.heads * HD + (size_t)h0 * HD;
  float *pmz = a.pmz + (cb * a.heads + h0) * 2;
  const uint32_t p0 = c * CS, pw = p0 + w * PW;
  const size_t slot = (size_t)b * a.kvheads + kvh;
  const uint16_t *kb = a.kc + slot * a.max_seq * HD;
  const uint16_t *vb = a.vc + slot * a.max_seq * HD;
  // ring: the stream position first (it fixes the ring's oldest slot)
  uint32_t rlen = 0, qrank = 0, woff = 0;
  if (RG) {
    const int32_t ps = a.pos[b];
    const uint32_t pos = ps < 0 ? 0u : (uint32_t)ps, cap = a.max_seq;
    rlen = pos + 1 < cap ? pos + 1 : cap;  // pos + 1 > 0: pos < 2^31
    const uint32_t start = pos >= cap ? pos - a.win + 1 : a.nsink;
    woff = (start - a.nsink) % a.win;
    qrank = pos < cap ? pos : cap - 1;
  }
  // a rank's slot: sink slot r below nsink, later ranks walk the ring from its oldest entry
  auto slot_of = [&](uint32_t pc) -> uint32_t {
    if (!RG || pc < a.nsink) return pc;
    const uint32_t t = woff + (pc - a.nsink);  // < 2 win
    return a.nsink + (t >= a.win ? t - a.win : t);
  };
  // q first (loads retire in issue order): lane (lg, li) takes head
  // h0 + li (li < 4; the others zero), dims 32 s + 8 lg .. + 7
  const float *qb = a.q + (size_t)qr * a.heads * HD + (size_t)(h0 + (li < G ? li : 0)) * HD + 8 * lg;
  float4 qv[8];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    qv[2 * s] = *(const float4 *)(qb + 32 * s);
    qv[2 * s + 1] = *(const float4 *)(qb + 32 * s + 4);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Rows past lim - 1 clamp to it.  Large caches (NT) read the position
  // first so that rows past it are never fetched; small ones fetch the whole
  // chunk while the position is in flight.
  uint32_t lim = a.max_seq, len = rlen;
  if (NT && !RG) {
    const int32_t pr = a.pos[0] + (a.qper ? (int32_t)(qr % a.qper) : 0);
    lim = (pr < 0 ? 0u : ((uint32_t)pr >= a.max_seq ? a.max_seq - 1 : (uint32_t)pr)) + 1;
    len = lim;  // positions attended: 0 .. pr
  }
  // K rows of the wave's 32 positions go straight into its tile (direct
  // global-to-LDS loads, whole rows per instruction: instruction k, lane
  // j = 16 rr + uu brings row 4 k + rr's 16-byte unit uu ^ (row % 16) to
  // tile unit uu of that row, so the A-operand reads below -- row 16 bb +
  // li, unit 4 s + lg -- hit 16 distinct units), read back in the matrix
  // cores' layout: lane (lg, li) position pw + 16 bb + li, dims 32 s + 8 lg.
  // (Fetched in that layout directly, each load instruction took a 64-byte
  // piece of 16 rows: 13.78 -> 13.25 us for the B = 32 pass.)  Large caches
  // stream K and V non-temporally, as k_attn_part does: with plain loads
  // the K rows evict what the step's linears re-read (measured at B = 32:
  // the pass alone 14.05 -> 14.25 us, the decode step 1.773 -> 1.713 ms).
  // (Ring caches keep K in registers, fetched in the A-operand layout
  // directly beside each row's rotation pairs: staged, that variant spills.)
  constexpr bool KLDS = !RG;
  uint8_t *const ktile = (uint8_t *)s_vt[w];
  uint4 kr[2][4];
  float4 rc[2][4], rs[2][4];  // ring: the rank's rotation pairs of the lane's 8 dims
  if (KLDS) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t row = 4 * k + (lane >> 4), uu = lane & 15;
      const uint32_t pp = pw + row, pc = pp < lim ? pp : lim - 1;
      __builtin_amdgcn_global_load_lds((const void *)(kb + (size_t)pc * HD + 8 * (uu ^ (row % 16))),
                                       (__attribute__((address_space(3))) void *)(ktile + 1024 * k), 16, 0,
                                       NT ? 2 : 0);  // aux 2: non-temporal
    }
    // every later load counts after these in vmcnt
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  } else {
#pragma unroll
    for (int bb = 0; bb < 2; bb++) {
      const uint32_t pp = pw + 16 * bb + li, pc = pp < lim ? pp : lim - 1;
      const size_t ro = (size_t)slot_of(pc) * HD;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        kr[bb][s] = kv_ld<NT>(kb + ro + 32 * s + 8 * lg);
        rc[bb][s] = *(const float4 *)(a.co + (size_t)pc * (HD / 2) + 16 * s + 4 * lg);
        rs[bb][s] = *(const float4 *)(a.si + (size_t)pc * (HD / 2) + 16 * s + 4 * lg);
      }
    }
  }
  // V, whole rows: lane (lg, li) positions pw + 16 u + 4 lg + r, dims 8 li .. + 7
  uint4 vr[2][4];
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t pp = pw + 16 * u + 4 * lg + r, pc = pp < lim ? pp : lim - 1;
      vr[u][r] = kv_ld<NT>(vb + (size_t)slot_of(pc) * HD + 8 * li);
    }
  // ring: q rotated by the query's rank (pairs 16 s + 4 lg + j of its dims)
  float4 qc[4], qs[4];
  if (RG) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      qc[s] = *(const float4 *)(a.co + (size_t)qrank * (HD / 2) + 16 * s + 4 * lg);
      qs[s] = *(const float4 *)(a.si + (size_t)qrank * (HD / 2) + 16 * s + 4 * lg);
    }
  }
  if (!RG && !NT) {
    const int32_t pr = a.pos[0] + (a.qper ? (int32_t)(qr % a.qper) : 0);
    len = (pr < 0 ? 0u : ((uint32_t)pr >= a.max_seq ? a.max_seq - 1 : (uint32_t)pr)) + 1;
  }
  if (p0 >= len) {  // block-uniform: a chunk past the position adds nothing
    // (the tile's direct loads land before the workgroup's LDS is released)
    if (KLDS) __builtin_amdgcn_s_waitcnt(0);
    for (int i = threadIdx.x; i < G * HD; i += NW * 64) pctx[i] = 0.0f;
    if (threadIdx.x < G) {
      pmz[2 * threadIdx.x] = -1.0e30f;
      pmz[2 * threadIdx.x + 1] = 0.0f;
    }
    return;
  }
  v8h qh[4], ql[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = li < G ? f4_at(qv[2 * s + e / 4], e % 4) : 0.0f;
    if (RG) {  // decode-attn-stream's rotation: C[i0] = a0*c - a1*s; C[i1] = a0*s + a1*c
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float x0 = x[2 * j], x1 = x[2 * j + 1], cj = f4_at(qc[s], j), sj = f4_at(qs[s], j);
        x[2 * j] = x0 * cj - x1 * sj;
        x[2 * j + 1] = x0 * sj + x1 * cj;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const _Float16 h = (_Float16)x[e];
      qh[s][e] = h;
      ql[s][e] = (_Float16)(x[e] - (float)h);
    }
  }
  if (KLDS) {
    // the tile's K loads have landed once at most the 8 V loads issued after
    // them are out: then read the A operands
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((8 & 0xF) | (0x7 << 4) | ((8 >> 4) << 14));
    asm volatile("" ::: "memory");
#pragma unroll
    for (int bb = 0; bb < 2; bb++)
#pragma unroll
      for (int s = 0; s < 4; s++)
        kr[bb][s] = *(const uint4 *)(ktile + (16 * bb + li) * 256 + 16 * ((4 * s + lg) ^ li));
  }
  // scores: lane (lg, li < 4) gets head li at positions pw + 16 bb + 4 lg + r
  v4f sc[2];
#pragma unroll
  for (int bb = 0; bb < 2; bb++) {
    sc[bb] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if (RG) {  // K rotated by its rank in f32, then hi + lo halves
        const v8h k16 = __builtin_bit_cast(v8h, kr[bb][s]);
        float kf32[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float k0 = (float)k16[2 * j], k1 = (float)k16[2 * j + 1];
          const float cj = f4_at(rc[bb][s], j), sj = f4_at(rs[bb][s], j);
          kf32[2 * j] = k0 * cj - k1 * sj;
          kf32[2 * j + 1] = k0 * sj + k1 * cj;
        }
        v8h kh, kl;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const _Float16 h = (_Float16)kf32[e];
          kh[e] = h;
          kl[e] = (_Float16)(kf32[e] - (float)h);
        }
        sc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[s], sc[bb], 0, 0, 0);
        sc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[s], sc[bb], 0, 0, 0);
        sc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[s], sc[bb], 0, 0, 0);
      } else {
        const v8h kf = __builtin_bit_cast(v8h, kr[bb][s]);
        sc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[s], sc[bb], 0, 0, 0);
        sc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[s], sc[bb], 0, 0, 0);
      }
    }
  }
  float m = -1.0e30f;
#pragma unroll
  for (int bb = 0; bb < 2; bb++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t pp = pw + 16 * bb + 4 * lg + r;
      sc[bb][r] = pp < len ? sc[bb][r] * a.coef : -INFINITY;  // (q.k / sqrt(hd)) * log2(e)
      m = sc[bb][r] > m ? sc[bb][r] : m;
    }
  // the head's maximum over the wave: lanes li, li + 16, li + 32, li + 48
  {
    float o = __shfl_xor(m, 16);
    m = o > m ? o : m;
    o = __shfl_xor(m, 32);
    m = o > m ? o : m;
  }
  float z = 0.0f;
  v8h ph, pl;
#pragma unroll
  for (int bb = 0; bb < 2; bb++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float e = nlg_exp2(sc[bb][r] - m);
      z = z + e;
      const _Float16 h = (_Float16)e;
      ph[4 * bb + r] = h;
      pl[4 * bb + r] = (_Float16)(e - (float)h);
    }
  z = z + __shfl_xor(z, 16);
  z = z + __shfl_xor(z, 32);
  // V^T tile: dims 8 li + e, slots 8 lg + 4 u + r (one wave's LDS operations
  // run in order, so the tile needs no barrier).  Rows past the position go
  // in as zeros: their probability is 0, but a cache row nobody wrote may
  // hold NaN or Inf bits, and 0 x NaN is NaN.
  uint16_t *vt = s_vt[w];
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int wd = e / 2, sh = 16 * (e & 1);
      uint32_t hv[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t word = wd == 0 ? vr[u][r].x : wd == 1 ? vr[u][r].y : wd == 2 ? vr[u][r].z : vr[u][r].w;
        hv[r] = (word >> sh) & (pw + 16 * u + 4 * lg + r < len ? 0xffffu : 0u);
      }
      *(uint2 *)&vt[(8 * li + e) * AMF_PITCH + 8 * lg + 4 * u] = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
    }
  // O^T = V^T P^T per 16-dim block n: lane (lg, li < 4) gets head li, dims 16 n + 4 lg + r
  v4f o[8];
#pragma unroll
  for (int n = 0; n < 8; n++) {
    const uint16_t *row = &vt[(16 * n + li) * AMF_PITCH + 8 * lg];
    const uint2 x0 = *(const uint2 *)row, x1 = *(const uint2 *)(row + 4);
    const v8h vf = __builtin_bit_cast(v8h, make_uint4(x0.x, x0.y, x1.x, x1.y));
    o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph, (v4f){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl, o[n], 0, 0, 0);
  }
  // the wave's context [G][HD] over its tile (every read of the tile above
  // feeds these values, so the stores follow them)
  float *ctxw = (float *)vt;
  if (li < G) {
#pragma unroll
    for (int n = 0; n < 8; n++) *(float4 *)&ctxw[li * HD + 16 * n + 4 * lg] = make_float4(o[n][0], o[n][1], o[n][2], o[n][3]);
    if (lg == 0) {
      s_m[w][li] = m;
      s_z[w][li] = z;
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * HD; idx += NW * 64) {
    const int h = idx / HD, d = idx % HD;
    float mm = s_m[0][h];
#pragma unroll
    for (int k = 1; k < NW; k++) mm = s_m[k][h] > mm ? s_m[k][h] : mm;
    float zz = 0.0f, cx = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; k++) {
      const float scl = nlg_exp2(s_m[k][h] - mm);
      zz = fmaf(s_z[k][h], scl, zz);
      cx = fmaf(((const float *)s_vt[k])[h * HD + d], scl, cx);
    }
    pctx[idx] = cx;
    if (d == 0) {
      pmz[2 * h] = mm;
      pmz[2 * h + 1] = zz;
    }
  }
}

// Pass 2: out = sum_c pctx_c * exp(m_c - M) / sum_c z_c * exp(m_c - M),
// M = max_c m_c, one thread per output element.
__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ pctx,
                                                    const float *__restrict__ pmz, float *__restrict__ out,
                                                    uint32_t batch, uint32_t heads, uint32_t hd,
                                                    uint32_t nchunk) {
  const uint32_t nh = heads * hd;
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)batch * nh) return;
  const uint32_t b = (uint32_t)(i / nh), e = (uint32_t)(i % nh), h = e / hd;
  const float *mz = pmz + ((size_t)b * nchunk * heads + h) * 2;
  const float *cx = pctx + (size_t)b * nchunk * nh + e;
  // chunks in groups of 8 whose loads are all issued together (addresses
  // clamped to the last chunk, weights of the extra ones zero)
  float mm = -1.0e30f;
  for (uint32_t c0 = 0; c0 < nchunk; c0 += 8) {
    float2 v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t c = c0 + k < nchunk ? c0 + k : nchunk - 1;
      v[k] = *(const float2 *)(mz + (size_t)c * heads * 2);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) mm = v[k].x > mm ? v[k].x : mm;
  }
  float zz = 0.0f, acc = 0.0f;
  for (uint32_t c0 = 0; c0 < nchunk; c0 += 8) {
    float2 v[8];
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t c = c0 + k < nchunk ? c0 + k : nchunk - 1;
      v[k] = *(const float2 *)(mz + (size_t)c * heads * 2);
      x[k] = cx[(size_t)c * nh];
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float sc = c0 + k < nchunk ? nlg_exp2(v[k].x - mm) : 0.0f;
      zz = fmaf(v[k].y, sc, zz);
      acc = fmaf(x[k], sc, acc);
    }
  }
  out[i] = acc / zz;
}

extern "C" size_t nlg_decode_attn_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                                uint32_t head_dim, uint32_t max_seq) {
  if (!kvheads || (head_dim != 64 && head_dim != 128) || !max_seq) return 0;
  const size_t nchunk = attn_chunks(head_dim, max_seq);
  const size_t ctx = (size_t)batch * nchunk * heads * head_dim * 4;
  return (ctx + 255) / 256 * 256 + (size_t)batch * nchunk * heads * 2 * 4;
}

// Validate and lay out the workspace; fills everything but q/kc/vc/pos.
static int attn_setup(AttnArgs &a, uint32_t batch, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                      uint32_t max_seq, void *workspace, size_t workspace_bytes) {
  if (!kvheads || !heads || heads % kvheads) return nlg_fail("decode attn: heads must be a multiple of kvheads");
  const uint32_t G = heads / kvheads;
  if (head_dim != 64 && head_dim != 128) return nlg_fail("decode attn: head_dim must be 64 or 128");
  if (G != 1 && G != 2 && G != 4 && G != 8) return nlg_fail("decode attn: heads/kvheads must be 1, 2, 4 or 8");
  if (!max_seq || batch > 65535 || kvheads > 65535) return nlg_fail("decode attn: bad max_seq/batch/kvheads");
  const size_t need = nlg_decode_attn_f16_workspace(batch, heads, kvheads, head_dim, max_seq);
  if (!workspace || workspace_bytes < need) return nlg_fail("decode attn: needs a %zu-byte workspace", need);
  a.nchunk = attn_chunks(head_dim, max_seq);
  const size_t ctx = (size_t)batch * a.nchunk * heads * head_dim * 4;
  a.pctx = (float *)workspace;
  a.pmz = (float *)((char *)workspace + (ctx + 255) / 256 * 256);
  a.heads = heads; a.kvheads = kvheads; a.max_seq = max_seq;
  a.coef = (1.0f / sqrtf((float)head_dim)) * NLG_LOG2E;  // (/ 1.0 (sqrt (float hd))), in base 2
  a.table = nullptr; a.lens = nullptr; a.bs = a.mbps = a.npool = 0;
  a.co = a.si = nullptr; a.nsink = a.win = 0;
  a.ent = nullptr; a.nslots = a.trows = 0;
  return NLG_OK;
}

// The chunk pass over `rows` query rows for a filled-in AttnArgs.  A
// workgroup scores every query head of its kv head (K and V read once)
// unless there are too few workgroups to spread over the CUs: then one head
// each (K and V come from L2 for the others).
static int attn_chunks_launch(AttnArgs &a, uint32_t rows, uint32_t head_dim, int mode, hipStream_t st) {
  const uint32_t ni = attn_ni(head_dim, a.max_seq);
  const uint32_t G = (uint64_t)rows * a.kvheads * a.nchunk >= 128 ? a.grp : 1;
  // positions attended per sequence at most: the cache (contiguous, ring) or
  // its block table's reach (paged); entry lists stay on plain loads
  const uint64_t seqs = a.qper ? (rows + a.qper - 1) / a.qper : rows;
  if (mode != AM_ENTRIES && seqs * a.kvheads * a.max_seq * head_dim * 4 >= ATTN_NT_BYTES) mode |= AM_NT;
  constexpr int AM_CONTIG_NT_ = AM_CONTIG | AM_NT;
  a.nunits = rows * a.kvheads * a.nchunk;
  const dim3 grid = G == 1 ? dim3((a.nunits + 7) / 8 * 8 * a.grp) : dim3(a.nchunk, a.heads / G, rows);
  const dim3 blk(ATTN_WAVES * 64);
  // (ring caches small enough for plain loads keep the VALU pass: that
  // variant's registers spill under the two-workgroups-per-CU bound)
  if (head_dim == 128 && G == 4 && ni == 8 &&
      ((mode & ~AM_NT) == AM_CONTIG || mode == (AM_RING | AM_NT))) {
    const bool nt = mode & AM_NT, rg = (mode & ~AM_NT) == AM_RING;
    if (rg) {
      hipLaunchKernelGGL((k_attn_mfma<true, true>), grid, blk, 0, st, a);
    } else {
      if (nt) hipLaunchKernelGGL((k_attn_mfma<true, false>), grid, blk, 0, st, a);
      else hipLaunchKernelGGL((k_attn_mfma<false, false>), grid, blk, 0, st, a);
    }
    NLG_LAUNCHED(rg ? "decode attention (ring fp16 KV, matrix cores)" : "decode attention (fp16 KV, matrix cores)");
    return NLG_OK;
  }
#define AT1(HD, GG, PGV)                                                                   \
  do {                                                                                     \
    if (ni == 8) hipLaunchKernelGGL((k_attn_part<HD, GG, 8, PGV>), grid, blk, 0, st, a);   \
    else hipLaunchKernelGGL((k_attn_part<HD, GG, 4, PGV>), grid, blk, 0, st, a);           \
  } while (0)
#define AT(HD, GG)                                                                         \
  do {                                                                                     \
    if (mode == AM_PAGED) AT1(HD, GG, AM_PAGED);                                           \
    else if (mode == (AM_PAGED | AM_NT)) AT1(HD, GG, AM_PAGED | AM_NT);                    \
    else if (mode == AM_RING) AT1(HD, GG, AM_RING);                                        \
    else if (mode == (AM_RING | AM_NT)) AT1(HD, GG, AM_RING | AM_NT);                      \
    else if (mode == AM_ENTRIES) AT1(HD, GG, AM_ENTRIES);                                  \
    else if (mode == AM_CONTIG_NT_) AT1(HD, GG, AM_CONTIG | AM_NT);                        \
    else AT1(HD, GG, AM_CONTIG);                                                           \
  } while (0)
  if (head_dim == 128) {
    if (G == 1) AT(128, 1); else if (G == 2) AT(128, 2); else if (G == 4) AT(128, 4); else AT(128, 8);
  } else {
    if (G == 1) AT(64, 1); else if (G == 2) AT(64, 2); else if (G == 4) AT(64, 4); else AT(64, 8);
  }
#undef AT
#undef AT1
  const int bm = mode & ~AM_NT;
  NLG_LAUNCHED(bm == AM_PAGED     ? "decode attention (paged fp16 KV)"
               : bm == AM_RING    ? "decode attention (ring fp16 KV)"
               : bm == AM_ENTRIES ? "decode attention (fp16 KV entry list)"
                                  : "decode attention (fp16 KV)");
  return NLG_OK;
}

int nlg_attn_chunks(const float *q, const uint16_t *kcache, const uint16_t *vcache, const int32_t *pos,
                    uint32_t rows, uint32_t qper, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                    uint32_t max_seq, void *workspace, size_t workspace_bytes, hipStream_t st) {
  if (!rows) return NLG_OK;
  AttnArgs a;
  if (attn_setup(a, rows, heads, kvheads, head_dim, max_seq, workspace, workspace_bytes)) return NLG_ERR;
  if (((uintptr_t)q & 15) || ((uintptr_t)kcache & 15) || ((uintptr_t)vcache & 15))
    return nlg_fail("decode attn: q and caches must be 16-byte aligned");
  a.q = q; a.kc = kcache; a.vc = vcache; a.pos = pos; a.qper = qper; a.grp = heads / kvheads;
  return attn_chunks_launch(a, rows, head_dim, AM_CONTIG, st);
}

extern "C" int nlg_decode_attn_f16_chunks(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                          const int32_t *pos, uint32_t batch, uint32_t heads,
                                          uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                                          void *workspace, size_t workspace_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  return nlg_attn_chunks(q, kcache, vcache, pos, batch, 0, heads, kvheads, head_dim, max_seq, workspace,
                         workspace_bytes, nlg_stream(stream));
}

extern "C" int nlg_attn_ternary_linear_residual(const void *workspace, size_t workspace_bytes, uint32_t batch,
                                                uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                                                uint32_t max_seq, const uint32_t *w2, const float *bias,
                                                const float *beta, int beta_per_row, const float *res,
                                                float *y, uint32_t out, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch) return NLG_OK;
  AttnArgs t;
  if (attn_setup(t, batch, heads, kvheads, head_dim, max_seq, (void *)workspace, workspace_bytes)) return NLG_ERR;
  if (t.nchunk > NLG_ATTN_MAX_CHUNKS)
    return nlg_fail("attention + linear: %u chunks (max_seq %u) exceed the %d the fused merge takes; "
                    "use nlg_decode_attn_f16 and nlg_ternary_linear_residual", t.nchunk, max_seq,
                    NLG_ATTN_MAX_CHUNKS);
  if (!res) return nlg_fail("attention + linear: res is null");
  FusedArgs a{};
  a.x = t.pctx; a.attn_mz = t.pmz; a.attn_nc = t.nchunk; a.hd = head_dim;
  a.w2 = w2; a.bias = bias; a.beta = beta; a.beta_per_row = beta_per_row;
  a.seq = batch; a.out = out; a.cols = heads * head_dim; a.y = y; a.ystride = out; a.res = res; a.rstride = out;
  return nlg_fused_launch(a, NLG_PRO_ATTN, NLG_EPI_RESID, 0, nlg_stream(stream));
}

// Paged fp16 caches: decode-attn-paged-v (kernels.el:1222-1246) over pools
// [block][bs][kvheads][head_dim] through the block table, each sequence at
// its own lens[b]; the same chunk pass and merge as the contiguous caches.
extern "C" size_t nlg_decode_attn_paged_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                                      uint32_t head_dim, uint32_t bs, uint32_t mbps) {
  const uint64_t ms = (uint64_t)bs * mbps;
  if (!ms || ms > 0xffffffffull) return 0;
  return nlg_decode_attn_f16_workspace(batch, heads, kvheads, head_dim, (uint32_t)ms);
}

extern "C" int nlg_decode_attn_paged_f16(const float *q, const uint16_t *kpool, const uint16_t *vpool,
                                         const int32_t *lens, const int32_t *table, uint32_t npool,
                                         float *out, uint32_t batch, uint32_t heads, uint32_t kvheads,
                                         uint32_t head_dim, uint32_t bs, uint32_t mbps, void *workspace,
                                         size_t workspace_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch) return NLG_OK;
  if (!q || !kpool || !vpool || !lens || !table || !out) return nlg_fail("paged attn: null pointer");
  if (!bs || !mbps || (uint64_t)bs * mbps > 0xffffffffull || !npool)
    return nlg_fail("paged attn: bad block size %u / blocks per sequence %u / pool %u", bs, mbps, npool);
  AttnArgs a;
  if (attn_setup(a, batch, heads, kvheads, head_dim, bs * mbps, workspace, workspace_bytes)) return NLG_ERR;
  if (((uintptr_t)q & 15) || ((uintptr_t)kpool & 15) || ((uintptr_t)vpool & 15))
    return nlg_fail("paged attn: q and pools must be 16-byte aligned");
  a.q = q; a.kc = kpool; a.vc = vpool; a.pos = lens; a.qper = 0; a.grp = heads / kvheads;
  a.table = table; a.lens = lens; a.bs = bs; a.mbps = mbps; a.npool = npool;
  hipStream_t st = nlg_stream(stream);
  if (attn_chunks_launch(a, batch, head_dim, AM_PAGED, st)) return NLG_ERR;
  const uint64_t n = (uint64_t)batch * heads * head_dim;
  hipLaunchKernelGGL(k_attn_merge, dim3(nlg_blocks(n, 256)), dim3(256), 0, st, a.pctx, a.pmz, out, batch,
                     heads, head_dim, a.nchunk);
  NLG_LAUNCHED("paged decode attention merge");
  return NLG_OK;
}

// Append B rows of K or V into a paged fp16 pool, row s at position lens[s]
// (cache-append-paged-v, kernels.el:1211-1220; fp16 round to nearest even).
__global__ __launch_bounds__(256) void k_append_paged_f16(const float *src, const int32_t *lens,
                                                          const int32_t *table, uint32_t npool, uint16_t *pool,
                                                          uint32_t batch, uint32_t kvdim, uint32_t bs,
                                                          uint32_t mbps) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)batch * kvdim) return;
  const uint32_t s = (uint32_t)(i / kvdim), t = (uint32_t)(i % kvdim);
  const int32_t pos = lens[s];
  if (pos < 0 || (uint64_t)pos >= (uint64_t)bs * mbps) return;
  const int32_t ph = table[(size_t)s * mbps + (uint32_t)pos / bs];
  if (ph < 0 || (uint32_t)ph >= npool) return;
  pool[((size_t)ph * bs + (uint32_t)pos % bs) * kvdim + t] = __builtin_bit_cast(uint16_t, (_Float16)src[i]);
}

extern "C" int nlg_cache_append_paged_f16(const float *src, const int32_t *lens, const int32_t *table,
                                          uint32_t npool, uint16_t *pool, uint32_t batch, uint32_t kvdim,
                                          uint32_t bs, uint32_t mbps, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch || !kvdim) return NLG_OK;
  if (!src || !lens || !table || !pool) return nlg_fail("paged append: null pointer");
  if (!bs || !mbps) return nlg_fail("paged append: block size and blocks per sequence must be nonzero");
  const uint64_t n = (uint64_t)batch * kvdim;
  hipLaunchKernelGGL(k_append_paged_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nlg_stream(stream), src,
                     lens, table, npool, pool, batch, kvdim, bs, mbps);
  NLG_LAUNCHED("paged fp16 append");
  return NLG_OK;
}

// StreamingLLM ring caches: decode-attn-stream (kernels.el:409-451) over
// fp16 caches [batch][kvheads][nsink + win][head_dim], each sequence at its
// own stream position pos[b]; the same chunk pass and merge as above.
extern "C" size_t nlg_decode_attn_stream_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                                      uint32_t head_dim, uint32_t nsink, uint32_t win) {
  const uint64_t cap = (uint64_t)nsink + win;
  if (!win || cap > 0x7fffffffull) return 0;
  return nlg_decode_attn_f16_workspace(batch, heads, kvheads, head_dim, (uint32_t)cap);
}

extern "C" int nlg_decode_attn_stream_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                          const int32_t *pos, const float *co, const float *si, float *out,
                                          uint32_t batch, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                                          uint32_t nsink, uint32_t win, void *workspace, size_t workspace_bytes,
                                          void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch) return NLG_OK;
  if (!q || !kcache || !vcache || !pos || !co || !si || !out) return nlg_fail("stream attn: null pointer");
  if (!win || (uint64_t)nsink + win > 0x7fffffffull)
    return nlg_fail("stream attn: win must be nonzero and nsink + win < 2^31 (nsink %u, win %u)", nsink, win);
  AttnArgs a;
  if (attn_setup(a, batch, heads, kvheads, head_dim, nsink + win, workspace, workspace_bytes)) return NLG_ERR;
  if (((uintptr_t)q & 15) || ((uintptr_t)kcache & 15) || ((uintptr_t)vcache & 15) || ((uintptr_t)co & 15) ||
      ((uintptr_t)si & 15))
    return nlg_fail("stream attn: q, caches and rotation tables must be 16-byte aligned");
  a.q = q; a.kc = kcache; a.vc = vcache; a.pos = pos; a.qper = 0; a.grp = heads / kvheads;
  a.co = co; a.si = si; a.nsink = nsink; a.win = win;
  hipStream_t st = nlg_stream(stream);
  if (attn_chunks_launch(a, batch, head_dim, AM_RING, st)) return NLG_ERR;
  const uint64_t n = (uint64_t)batch * heads * head_dim;
  hipLaunchKernelGGL(k_attn_merge, dim3(nlg_blocks(n, 256)), dim3(256), 0, st, a.pctx, a.pmz, out, batch,
                     heads, head_dim, a.nchunk);
  NLG_LAUNCHED("ring decode attention merge");
  return NLG_OK;
}

// attn-stream-entries (kernels.el:1052-1090) over fp16 caches
// [batch][kvheads][nslots][head_dim]: sequence b attends the ne rows its
// entry list ent[b] names, (slot, cache-relative rank) int32 pairs, K rotated
// by the rank and q by qrank[b]; tables co/si hold trows rows.
extern "C" size_t nlg_attn_entries_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                                 uint32_t head_dim, uint32_t ne) {
  return nlg_decode_attn_f16_workspace(batch, heads, kvheads, head_dim, ne);
}

extern "C" int nlg_attn_entries_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                    const int32_t *ent, const int32_t *qrank, const float *co, const float *si,
                                    float *out, uint32_t batch, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                                    uint32_t nslots, uint32_t ne, uint32_t trows, void *workspace,
                                    size_t workspace_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch) return NLG_OK;
  if (!q || !kcache || !vcache || !ent || !qrank || !co || !si || !out) return nlg_fail("entries attn: null pointer");
  if (!nslots || !ne || !trows) return nlg_fail("entries attn: nslots, ne and trows must be nonzero");
  AttnArgs a;
  if (attn_setup(a, batch, heads, kvheads, head_dim, ne, workspace, workspace_bytes)) return NLG_ERR;
  if (((uintptr_t)q & 15) || ((uintptr_t)kcache & 15) || ((uintptr_t)vcache & 15) || ((uintptr_t)co & 15) ||
      ((uintptr_t)si & 15) || ((uintptr_t)ent & 7))
    return nlg_fail("entries attn: q, caches and tables must be 16-byte aligned, ent 8-byte aligned");
  a.q = q; a.kc = kcache; a.vc = vcache; a.pos = qrank; a.lens = qrank; a.qper = 0; a.grp = heads / kvheads;
  a.co = co; a.si = si; a.ent = ent; a.nslots = nslots; a.trows = trows;
  hipStream_t st = nlg_stream(stream);
  if (attn_chunks_launch(a, batch, head_dim, AM_ENTRIES, st)) return NLG_ERR;
  const uint64_t n = (uint64_t)batch * heads * head_dim;
  hipLaunchKernelGGL(k_attn_merge, dim3(nlg_blocks(n, 256)), dim3(256), 0, st, a.pctx, a.pmz, out, batch,
                     heads, head_dim, a.nchunk);
  NLG_LAUNCHED("entry-list decode attention merge");
  return NLG_OK;
}

// block-copy (kernels.el:1184-1193) for both fp16 pools at once, n copies in
// one launch: pair i = (src block, dst block) of pairs[2i..2i+1]; pairs with
// a block outside [0, npool) are skipped.  A workgroup copies one block of
// bs * kvdim halves in 16-byte pieces when kvdim % 8 == 0, else halves.
template <bool V16>
__global__ __launch_bounds__(256) void k_block_copy_f16(uint16_t *kpool, uint16_t *vpool, const int32_t *pairs,
                                                        uint32_t npool, uint32_t bn) {
  const int32_t src = pairs[2 * blockIdx.x], dst = pairs[2 * blockIdx.x + 1];
  if (src < 0 || dst < 0 || (uint32_t)src >= npool || (uint32_t)dst >= npool) return;
  if (V16) {
    const uint32_t n16 = bn / 8;
    const uint4 *ks = (const uint4 *)(kpool + (size_t)src * bn), *vs = (const uint4 *)(vpool + (size_t)src * bn);
    uint4 *kd = (uint4 *)(kpool + (size_t)dst * bn), *vd = (uint4 *)(vpool + (size_t)dst * bn);
    for (uint32_t i = threadIdx.x; i < n16; i += 256) {
      kd[i] = ks[i];
      vd[i] = vs[i];
    }
  } else {
    for (uint32_t i = threadIdx.x; i < bn; i += 256) {
      kpool[(size_t)dst * bn + i] = kpool[(size_t)src * bn + i];
      vpool[(size_t)dst * bn + i] = vpool[(size_t)src * bn + i];
    }
  }
}

extern "C" int nlg_block_copy_f16(uint16_t *kpool, uint16_t *vpool, const int32_t *pairs, uint32_t n,
                                  uint32_t npool, uint32_t bs, uint32_t kvdim, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!n || !bs || !kvdim) return NLG_OK;
  if (!kpool || !vpool || !pairs) return nlg_fail("block copy: null pointer");
  if (n > 0x7fffffffu || (uint64_t)bs * kvdim > 0xffffffffull) return nlg_fail("block copy: too many copies or too large a block");
  const uint32_t bn = bs * kvdim;
  const bool v16 = kvdim % 8 == 0 && !((uintptr_t)kpool & 15) && !((uintptr_t)vpool & 15);
  if (v16) hipLaunchKernelGGL(k_block_copy_f16<true>, dim3(n), dim3(256), 0, nlg_stream(stream), kpool, vpool, pairs,
                              npool, bn);
  else hipLaunchKernelGGL(k_block_copy_f16<false>, dim3(n), dim3(256), 0, nlg_stream(stream), kpool, vpool, pairs,
                          npool, bn);
  NLG_LAUNCHED("fp16 block copy");
  return NLG_OK;
}

// Append B raw (un-rotated) rows of K or V into fp16 ring caches, row s at
// the slot of stream position pos[s] (cache-append-ring, kernels.el:396-407:
// slot = pos < nsink ? pos : nsink + (pos - nsink) mod win; fp16 round to
// nearest even).  Negative positions write nothing.
__global__ __launch_bounds__(256) void k_append_ring_f16(const float *src, const int32_t *pos, uint16_t *cache,
                                                         uint32_t batch, uint32_t kvheads, uint32_t hd,
                                                         uint32_t nsink, uint32_t win) {
  const uint32_t kvdim = kvheads * hd;
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)batch * kvdim) return;
  const uint32_t s = (uint32_t)(i / kvdim), t = (uint32_t)(i % kvdim);
  const int32_t p = pos[s];
  if (p < 0) return;
  const uint32_t slot = (uint32_t)p < nsink ? (uint32_t)p : nsink + ((uint32_t)p - nsink) % win;
  const size_t row = (size_t)s * kvheads + t / hd;
  cache[(row * (nsink + win) + slot) * hd + t % hd] = __builtin_bit_cast(uint16_t, (_Float16)src[i]);
}

extern "C" int nlg_cache_append_ring_f16(const float *src, const int32_t *pos, uint16_t *cache, uint32_t batch,
                                         uint32_t kvheads, uint32_t head_dim, uint32_t nsink, uint32_t win,
                                         void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch || !kvheads || !head_dim) return NLG_OK;
  if (!src || !pos || !cache) return nlg_fail("ring append: null pointer");
  if (!win || (uint64_t)nsink + win > 0x7fffffffull)
    return nlg_fail("ring append: win must be nonzero and nsink + win < 2^31 (nsink %u, win %u)", nsink, win);
  const uint64_t n = (uint64_t)batch * kvheads * head_dim;
  hipLaunchKernelGGL(k_append_ring_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nlg_stream(stream), src,
                     pos, cache, batch, kvheads, head_dim, nsink, win);
  NLG_LAUNCHED("ring fp16 append");
  return NLG_OK;
}

extern "C" int nlg_decode_attn_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                   const int32_t *pos, float *out, uint32_t batch, uint32_t heads,
                                   uint32_t kvheads, uint32_t head_dim, uint32_t max_seq,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!batch) return NLG_OK;
  if (nlg_decode_attn_f16_chunks(q, kcache, vcache, pos, batch, heads, kvheads, head_dim, max_seq, workspace,
                                 workspace_bytes, stream))
    return NLG_ERR;
  AttnArgs a;
  attn_setup(a, batch, heads, kvheads, head_dim, max_seq, workspace, workspace_bytes);
  hipStream_t st = nlg_stream(stream);
  const uint64_t n = (uint64_t)batch * heads * head_dim;
  hipLaunchKernelGGL(k_attn_merge, dim3(nlg_blocks(n, 256)), dim3(256), 0, st, a.pctx, a.pmz, out, batch,
                     heads, head_dim, a.nchunk);
  NLG_LAUNCHED("decode attention merge");
  return NLG_OK;
}
