// nlg_elem.hip -- elementwise and glue kernels of the hot path.
//
// These are one-invocation-per-element kernels in the reference and stay so
// here (they are HBM-bound and trivially coalesced).  Their bodies follow
// lisp/nelisp-gpu-kernels.el line by line (cited per body) and access memory
// robustly: a read past a buffer's end gives 0 and a write past it is
// dropped, which is what a Vulkan robustBufferAccess device does with the
// same request, so data-dependent indices (POS, TOK, wbase) can never fault
// the GPU.  Arithmetic is single IEEE operations in body order (the library
// is built with -ffp-contract=off), so everything not involving exp/pow/
// sin/cos is bit-identical to the CPU restatement.
#include "nlg_internal.h"

struct RB {
  float *p;
  uint32_t n;
};
struct EArgs {
  RB b[6];
  uint32_t p[5];
  uint32_t n;  // invocations that run: min(domain, 64*groups)
};

__device__ __forceinline__ float rld(const RB &b, uint32_t i) { return i < b.n ? b.p[i] : 0.0f; }
__device__ __forceinline__ void rst(const RB &b, uint32_t i, float v) {
  if (i < b.n) b.p[i] = v;
}
__device__ __forceinline__ uint32_t udiv(uint32_t a, uint32_t b) { return b ? a / b : 0u; }
__device__ __forceinline__ uint32_t umod(uint32_t a, uint32_t b) { return b ? a % b : 0u; }

#define NEG_BIG (-1.0e30f)
#define A(i) a.b[i]
#define P(i) a.p[i]

// vadd (kernels.el:12-16), add2 (:812-821)
__device__ void b_add(const EArgs &a, uint32_t i) {
  if (i < P(0)) rst(A(2), i, __fadd_rn(rld(A(0), i), rld(A(1), i)));
}
// mul (:1322-1324)
__device__ void b_mul(const EArgs &a, uint32_t i) {
  if (i < P(0)) rst(A(2), i, __fmul_rn(rld(A(0), i), rld(A(1), i)));
}
// scale (:141-146)
__device__ void b_scale(const EArgs &a, uint32_t i) {
  if (i < P(0)) rst(A(2), i, __fmul_rn(rld(A(0), i), rld(A(1), 0)));
}
// causal-mask (:148-155)
__device__ void b_causal_mask(const EArgs &a, uint32_t idx) {
  const uint32_t Nn = P(0);
  if (idx < Nn * Nn) {
    const uint32_t i = udiv(idx, Nn), j = umod(idx, Nn);
    if (j > i) rst(A(0), idx, NEG_BIG);
  }
}
// silu (:1306-1312)
__device__ void b_silu(const EArgs &a, uint32_t i) {
  if (i < P(0)) {
    const float x = rld(A(0), i);
    const float sg = 1.0f / __fadd_rn(1.0f, expf(__fsub_rn(0.0f, x)));
    rst(A(1), i, __fmul_rn(x, sg));
  }
}
// silu-mul (:186-193)
__device__ void b_silu_mul(const EArgs &a, uint32_t i) {
  if (i < P(0)) {
    const float x = rld(A(0), i);
    const float sg = 1.0f / __fadd_rn(1.0f, expf(__fsub_rn(0.0f, x)));
    rst(A(2), i, __fmul_rn(__fmul_rn(x, sg), rld(A(1), i)));
  }
}
// rmsnorm-fwd (:1258-1265)
__device__ void b_rmsnorm_fwd(const EArgs &a, uint32_t idx) {
  const uint32_t M = P(0), N = P(1);
  if (idx < M * N) {
    const uint32_t r = udiv(idx, N), j = umod(idx, N);
    rst(A(3), idx, __fmul_rn(__fmul_rn(rld(A(0), idx), rld(A(1), r)), rld(A(2), j)));
  }
}
// embed-gather (:1382-1392)
__device__ void b_embed_gather(const EArgs &a, uint32_t idx) {
  const uint32_t seq = P(0), dim = P(1);
  if (idx < seq * dim) {
    const uint32_t i = udiv(idx, dim), j = umod(idx, dim);
    const uint32_t tk = nlg_f2u(rld(A(0), i));
    rst(A(2), idx, rld(A(1), tk * dim + j));
  }
}
// cache-append (:307-314)
__device__ void b_cache_append(const EArgs &a, uint32_t idx) {
  const uint32_t kvdim = P(0);
  if (idx < kvdim) {
    const uint32_t pos = nlg_f2u(rld(A(1), 0));
    rst(A(2), pos * kvdim + idx, rld(A(0), idx));
  }
}
// cache-append-b (:356-365)
__device__ void b_cache_append_b(const EArgs &a, uint32_t idx) {
  const uint32_t B = P(0), kvdim = P(1), maxseq = P(2);
  if (idx < B * kvdim) {
    const uint32_t bb = udiv(idx, kvdim), t = umod(idx, kvdim);
    const uint32_t pos = nlg_f2u(rld(A(1), 0));
    rst(A(2), (bb * maxseq + pos) * kvdim + t, rld(A(0), idx));
  }
}
// qkv-append (:1042-1050)
__device__ void b_qkv_append(const EArgs &a, uint32_t idx) {
  const uint32_t dim = P(0), kvdim = P(1), wbase = P(2);
  if (idx < kvdim) {
    rst(A(1), wbase + idx, rld(A(0), dim + idx));
    rst(A(2), wbase + idx, rld(A(0), dim + (kvdim + idx)));
  }
}
// cache-append-ring (:396-403): SRC POS CACHE; push (kvdim nsink win).
// Stream position pos lives in slot pos (a sink) or nsink + (pos-nsink) % win.
__device__ void b_cache_append_ring(const EArgs &a, uint32_t idx) {
  const uint32_t kvdim = P(0), nsink = P(1), win = P(2);
  if (idx < kvdim) {
    const uint32_t pos = nlg_f2u(rld(A(1), 0));
    uint32_t slot = pos;
    if (pos >= nsink) slot = nsink + umod(pos - nsink, win);
    rst(A(2), slot * kvdim + idx, rld(A(0), idx));
  }
}
// cache-append-paged (:1099-1108) / -v (:1211-1220): SRC POS|LENS TABLE POOL;
// push (B kvdim bs mbps).  Row s goes to block TABLE[s*mbps + pos/bs],
// offset pos % bs, at the shared POS[0] or at its own LENS[s].
template <bool PER_SEQ>
__device__ void b_cache_append_paged(const EArgs &a, uint32_t idx) {
  const uint32_t B = P(0), kvdim = P(1), bs = P(2), mbps = P(3);
  if (idx < B * kvdim) {
    const uint32_t s = udiv(idx, kvdim), t = umod(idx, kvdim);
    const uint32_t pos = nlg_f2u(rld(A(1), PER_SEQ ? s : 0u));
    const uint32_t lb = udiv(pos, bs), off = umod(pos, bs);
    const uint32_t phys = nlg_f2u(rld(A(2), s * mbps + lb));
    rst(A(3), (phys * bs + off) * kvdim + t, rld(A(0), idx));
  }
}
// block-copy (:1182-1189): POOL; push (bs kvdim src dst) -- block src to
// block dst of the same pool (distinct blocks never overlap; src == dst
// rewrites each element with itself).
__device__ void b_block_copy(const EArgs &a, uint32_t i) {
  const uint32_t bs = P(0), kvdim = P(1), src = P(2), dst = P(3);
  const uint32_t bn = bs * kvdim;
  if (i < bn) rst(A(0), dst * bn + i, rld(A(0), src * bn + i));
}
// The rotation shared by the table-driven RoPE kernels.
__device__ __forceinline__ void rot_pair(const EArgs &a, int ix, int ic, int is, int isg, int ic_out,
                                         uint32_t ci, uint32_t i0, uint32_t i1) {
  const float cc = rld(A(ic), ci), ss = __fmul_rn(rld(A(is), ci), rld(A(isg), 0));
  const float a0 = rld(A(ix), i0), a1 = rld(A(ix), i1);
  rst(A(ic_out), i0, __fsub_rn(__fmul_rn(a0, cc), __fmul_rn(a1, ss)));
  rst(A(ic_out), i1, __fadd_rn(__fmul_rn(a0, ss), __fmul_rn(a1, cc)));
}
// decode-rope (:291-306): X CO SI SG POS C; push (cols heads)
__device__ void b_decode_rope(const EArgs &a, uint32_t idx) {
  const uint32_t cols = P(0), heads = P(1);
  const uint32_t hd = udiv(cols, heads), half = udiv(hd, 2);
  if (idx < heads * half) {
    const uint32_t m = umod(idx, half), h = udiv(idx, half);
    const uint32_t pos = nlg_f2u(rld(A(4), 0)), ci = pos * half + m;
    const uint32_t i0 = h * hd + 2 * m;
    rot_pair(a, 0, 1, 2, 3, 5, ci, i0, i0 + 1);
  }
}
// decode-rope-b (:340-355): push (B cols heads)
__device__ void b_decode_rope_b(const EArgs &a, uint32_t idx) {
  const uint32_t B = P(0), cols = P(1), heads = P(2);
  const uint32_t hd = udiv(cols, heads), half = udiv(hd, 2), rh = heads * half;
  if (idx < B * rh) {
    const uint32_t bb = udiv(idx, rh), rem = umod(idx, rh);
    const uint32_t m = umod(rem, half), h = udiv(rem, half);
    const uint32_t pos = nlg_f2u(rld(A(4), 0)), ci = pos * half + m;
    const uint32_t i0 = (bb * cols + h * hd) + 2 * m;
    rot_pair(a, 0, 1, 2, 3, 5, ci, i0, i0 + 1);
  }
}
// decode-rope-b-v (:1195-1209): X CO SI SG LENS C; push (B cols heads) --
// decode-rope-b with row bb rotated at its own position LENS[bb]
__device__ void b_decode_rope_b_v(const EArgs &a, uint32_t idx) {
  const uint32_t B = P(0), cols = P(1), heads = P(2);
  const uint32_t hd = udiv(cols, heads), half = udiv(hd, 2), rh = heads * half;
  if (idx < B * rh) {
    const uint32_t bb = udiv(idx, rh), rem = umod(idx, rh);
    const uint32_t m = umod(rem, half), h = udiv(rem, half);
    const uint32_t pos = nlg_f2u(rld(A(4), bb)), ci = pos * half + m;
    const uint32_t i0 = (bb * cols + h * hd) + 2 * m;
    rot_pair(a, 0, 1, 2, 3, 5, ci, i0, i0 + 1);
  }
}
// rope-apply (:1288-1304): X CO SI SG C; push (seq dim heads)
__device__ void b_rope_apply(const EArgs &a, uint32_t idx) {
  const uint32_t seq = P(0), dim = P(1), heads = P(2);
  const uint32_t hd = udiv(dim, heads), half = udiv(hd, 2);
  if (idx < (seq * heads) * half) {
    const uint32_t m = umod(idx, half), tmp = udiv(idx, half);
    const uint32_t h = umod(tmp, heads), p = udiv(tmp, heads);
    const uint32_t ci = p * half + m, i0 = (p * dim + h * hd) + 2 * m;
    rot_pair(a, 0, 1, 2, 3, 4, ci, i0, i0 + 1);
  }
}
// rope-half (:844-882): X Y; push (seq nheads hd rbase sgn), rbase/sgn are
// f32 bit patterns.  cos/sin/pow are the device library's (tolerance parity).
__device__ void b_rope_half(const EArgs &a, uint32_t idx) {
  const uint32_t seq = P(0), nheads = P(1), hd = P(2);
  const float rbase = __uint_as_float(P(3)), sgn = __uint_as_float(P(4));
  const uint32_t half = udiv(hd, 2);
  if (idx < (seq * nheads) * half) {
    const uint32_t m = umod(idx, half), tmp = udiv(idx, half);
    const uint32_t h = umod(tmp, nheads), p = udiv(tmp, nheads);
    const uint32_t b0 = p * (nheads * hd) + h * hd;
    const float ex = __fmul_rn(2.0f, (float)m) / (float)hd;
    const float theta = (float)p / powf(rbase, ex);
    const float c = cosf(theta), s = __fmul_rn(sgn, sinf(theta));
    const float a0 = rld(A(0), b0 + m), a1 = rld(A(0), b0 + (m + half));
    rst(A(1), b0 + m, __fsub_rn(__fmul_rn(a0, c), __fmul_rn(a1, s)));
    rst(A(1), b0 + (m + half), __fadd_rn(__fmul_rn(a1, c), __fmul_rn(a0, s)));
  }
}

template <void (*BODY)(const EArgs &, uint32_t)>
__global__ __launch_bounds__(256) void k_elem(EArgs a) {
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) BODY(a, i);
}

template <void (*BODY)(const EArgs &, uint32_t)>
static int elem(const nlg_buffer *b, int nbuf, const uint32_t *p, int npush, uint32_t domain,
                uint32_t groups, hipStream_t st, const char *name) {
  EArgs a;
  for (int i = 0; i < 6; i++) a.b[i] = RB{i < nbuf ? (float *)b[i].ptr : nullptr, i < nbuf ? b[i].nfloats : 0u};
  for (int i = 0; i < 5; i++) a.p[i] = i < npush ? p[i] : 0u;
  const uint64_t n = nlg_domain(domain, groups);
  if (!n) return NLG_OK;
  a.n = (uint32_t)n;
  uint32_t grid = nlg_blocks(n, 256);
  const uint32_t cap = (uint32_t)nlg_num_cu() * 32u;
  if (cap && grid > cap) grid = cap;
  hipLaunchKernelGGL(k_elem<BODY>, dim3(grid), dim3(256), 0, st, a);
  NLG_LAUNCHED(name);
  return NLG_OK;
}

#define E(fn, body, nb, np, dom)                                                          \
  int fn(const nlg_buffer *b, const uint32_t *p, uint32_t groups, hipStream_t st) {       \
    return elem<body>(b, nb, p, np, (dom), groups, st, #fn);                              \
  }

E(L_vadd, b_add, 3, 1, p[0])
E(L_add2, b_add, 3, 1, p[0])
E(L_mul, b_mul, 3, 1, p[0])
E(L_scale, b_scale, 3, 1, p[0])
E(L_causal_mask, b_causal_mask, 1, 1, p[0] * p[0])
E(L_silu, b_silu, 2, 1, p[0])
E(L_silu_mul, b_silu_mul, 3, 1, p[0])
E(L_rmsnorm_fwd, b_rmsnorm_fwd, 4, 2, p[0] * p[1])
E(L_embed_gather, b_embed_gather, 3, 2, p[0] * p[1])
E(L_cache_append, b_cache_append, 3, 1, p[0])
E(L_cache_append_b, b_cache_append_b, 3, 3, p[0] * p[1])
E(L_qkv_append, b_qkv_append, 3, 3, p[1])
E(L_decode_rope, b_decode_rope, 6, 2, (p[1] * ((p[1] ? p[0] / p[1] : 0u) / 2u)))
E(L_decode_rope_b, b_decode_rope_b, 6, 3, p[0] * (p[2] * ((p[2] ? p[1] / p[2] : 0u) / 2u)))
E(L_rope_apply, b_rope_apply, 5, 3, (p[0] * p[2]) * ((p[2] ? p[1] / p[2] : 0u) / 2u))
E(L_decode_rope_b_v, b_decode_rope_b_v, 6, 3, p[0] * (p[2] * ((p[2] ? p[1] / p[2] : 0u) / 2u)))
E(L_cache_append_ring, b_cache_append_ring, 3, 3, p[0])
E(L_cache_append_paged, b_cache_append_paged<false>, 4, 4, p[0] * p[1])
E(L_cache_append_paged_v, b_cache_append_paged<true>, 4, 4, p[0] * p[1])
E(L_block_copy, b_block_copy, 1, 4, p[0] * p[1])
E(L_rope_half, b_rope_half, 2, 5, (p[0] * p[1]) * (p[2] / 2u))
