/* nlg_oracle.c -- CPU restatement of nelisp-gpu's hot-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see nlg_oracle.h).  Never part of the product.
 *
 * Every kernel below restates the per-invocation DSL body of the cited
 * entry in lisp/nelisp-gpu-kernels.el ("kernels.el:LINE"), statement for
 * statement, with the op semantics of lisp/nelisp-gpu-compile.el:
 *   - uint `+ - * / %` wrap mod 2^32 (compile.el:176-183, OpIAdd/OpUDiv ...);
 *     a division by zero yields 0 here (undefined in SPIR-V, never exercised);
 *   - float compares are ordered, so NaN compares false (compile.el:185-191);
 *   - `(uint f)` is OpConvertFToS into a uint (compile.el:327): truncation
 *     toward zero; NaN gives 0 and out-of-range saturates (SPIR-V leaves those
 *     undefined; this is the convention the GPU build follows too);
 *   - `sdot` is a signed 4x8-bit dot product, lane i = byte i (compile.el:306-310);
 *   - exp/sqrt/sin/cos/pow are the C library's single-precision functions
 *     (the reference's are the Vulkan driver's GLSL.std.450 ones, so results
 *     that pass through them are pinned by tolerance, never bitwise).
 * Floats are evaluated one IEEE operation at a time in body order; the file is
 * compiled with -ffp-contract=off and without -ffast-math.
 */
#include "nlg_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
  float **b;
  const uint32_t *n;
  const uint32_t *p;
  uint32_t nthreads;
} K;

static inline float ld(const K *k, int bi, uint32_t i) { return i < k->n[bi] ? k->b[bi][i] : 0.0f; }
static inline uint32_t f2bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t ldu(const K *k, int bi, uint32_t i) { return f2bits(ld(k, bi, i)); }
static inline void st(const K *k, int bi, uint32_t i, float v) {
  if (i < k->n[bi]) k->b[bi][i] = v;
}
static inline uint32_t udiv(uint32_t a, uint32_t b) { return b ? a / b : 0u; }
static inline uint32_t umod(uint32_t a, uint32_t b) { return b ? a % b : 0u; }
/* (uint f): OpConvertFToS with a uint result type (compile.el:327). */
static inline uint32_t f2u(float f) {
  if (!(f == f)) return 0u;
  if (f >= 2147483648.0f) return 0x7fffffffu;
  if (f <= -2147483648.0f) return 0x80000000u;
  return (uint32_t)(int32_t)f;
}
/* OpSDot, PackedVectorFormat4x8Bit: signed bytes, lane i = byte i. */
static inline int32_t sdot4(uint32_t a, uint32_t b) {
  int32_t s = 0;
  for (int i = 0; i < 4; i++) s += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
  return s;
}
/* int32 add with two's-complement wrap (OpIAdd on :int). */
static inline int32_t iadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
/* f32 constant 1e-6 as the DSL compiles `0.000001` (compile.el:120-156). */
#define EPS6 0.000001f
#define NEG_BIG (-1.0e30f)

#define P(i) (k->p[i])

/* ---- elementwise ------------------------------------------------------ */

/* vadd, kernels.el:12-16 */
static void kn_vadd(const K *k, uint32_t i) {
  if (i < P(0)) st(k, 2, i, ld(k, 0, i) + ld(k, 1, i));
}
/* add2, kernels.el:816-821 */
static void kn_add2(const K *k, uint32_t i) {
  if (i < P(0)) st(k, 2, i, ld(k, 0, i) + ld(k, 1, i));
}
/* mul, kernels.el:1322-1324 */
static void kn_mul(const K *k, uint32_t i) {
  if (i < P(0)) st(k, 2, i, ld(k, 0, i) * ld(k, 1, i));
}
/* scale, kernels.el:141-146 */
static void kn_scale(const K *k, uint32_t i) {
  if (i < P(0)) st(k, 2, i, ld(k, 0, i) * ld(k, 1, 0));
}
/* causal-mask, kernels.el:148-155 */
static void kn_causal_mask(const K *k, uint32_t idx) {
  uint32_t Nn = P(0);
  if (idx < Nn * Nn) {
    uint32_t i = udiv(idx, Nn), j = umod(idx, Nn);
    if (j > i) st(k, 0, idx, NEG_BIG);
  }
}
/* silu-mul, kernels.el:186-193 */
static void kn_silu_mul(const K *k, uint32_t i) {
  if (i < P(0)) {
    float a = ld(k, 0, i);
    float sg = 1.0f / (1.0f + expf(0.0f - a));
    st(k, 2, i, (a * sg) * ld(k, 1, i));
  }
}
/* silu, kernels.el:1306-1312 */
static void kn_silu(const K *k, uint32_t i) {
  if (i < P(0)) {
    float x = ld(k, 0, i);
    float sg = 1.0f / (1.0f + expf(0.0f - x));
    st(k, 1, i, x * sg);
  }
}
/* rmsnorm-fwd, kernels.el:1258-1265 */
static void kn_rmsnorm_fwd(const K *k, uint32_t idx) {
  uint32_t M = P(0), N = P(1);
  if (idx < M * N) {
    uint32_t r = udiv(idx, N), j = umod(idx, N);
    st(k, 3, idx, (ld(k, 0, idx) * ld(k, 1, r)) * ld(k, 2, j));
  }
}
/* embed-gather, kernels.el:1382-1392 */
static void kn_embed_gather(const K *k, uint32_t idx) {
  uint32_t seq = P(0), dim = P(1);
  if (idx < seq * dim) {
    uint32_t i = udiv(idx, dim), j = umod(idx, dim);
    uint32_t tk = f2u(ld(k, 0, i));
    st(k, 2, idx, ld(k, 1, tk * dim + j));
  }
}
/* cache-append, kernels.el:307-314 */
static void kn_cache_append(const K *k, uint32_t idx) {
  uint32_t kvdim = P(0);
  if (idx < kvdim) {
    uint32_t pos = f2u(ld(k, 1, 0));
    st(k, 2, pos * kvdim + idx, ld(k, 0, idx));
  }
}
/* cache-append-b, kernels.el:356-365 */
static void kn_cache_append_b(const K *k, uint32_t idx) {
  uint32_t B = P(0), kvdim = P(1), maxseq = P(2);
  if (idx < B * kvdim) {
    uint32_t bb = udiv(idx, kvdim), t = umod(idx, kvdim);
    uint32_t pos = f2u(ld(k, 1, 0));
    st(k, 2, (bb * maxseq + pos) * kvdim + t, ld(k, 0, idx));
  }
}
/* qkv-append, kernels.el:1042-1050 */
static void kn_qkv_append(const K *k, uint32_t idx) {
  uint32_t dim = P(0), kvdim = P(1), wbase = P(2);
  if (idx < kvdim) {
    st(k, 1, wbase + idx, ld(k, 0, dim + idx));
    st(k, 2, wbase + idx, ld(k, 0, dim + (kvdim + idx)));
  }
}

/* ---- rotary ----------------------------------------------------------- */

/* decode-rope, kernels.el:291-306 */
static void kn_decode_rope(const K *k, uint32_t idx) {
  uint32_t cols = P(0), heads = P(1);
  uint32_t hd = udiv(cols, heads), half = udiv(hd, 2);
  if (idx < heads * half) {
    uint32_t m = umod(idx, half), h = udiv(idx, half);
    uint32_t pos = f2u(ld(k, 4, 0)), ci = pos * half + m;
    float cc = ld(k, 1, ci), ss = ld(k, 2, ci) * ld(k, 3, 0);
    uint32_t b0 = h * hd, i0 = b0 + 2 * m, i1 = i0 + 1;
    float a0 = ld(k, 0, i0), a1 = ld(k, 0, i1);
    st(k, 5, i0, (a0 * cc) - (a1 * ss));
    st(k, 5, i1, (a0 * ss) + (a1 * cc));
  }
}
/* decode-rope-b, kernels.el:340-355 */
static void kn_decode_rope_b(const K *k, uint32_t idx) {
  uint32_t B = P(0), cols = P(1), heads = P(2);
  uint32_t hd = udiv(cols, heads), half = udiv(hd, 2), rh = heads * half;
  if (idx < B * rh) {
    uint32_t bb = udiv(idx, rh), rem = umod(idx, rh);
    uint32_t m = umod(rem, half), h = udiv(rem, half);
    uint32_t pos = f2u(ld(k, 4, 0)), ci = pos * half + m;
    float cc = ld(k, 1, ci), ss = ld(k, 2, ci) * ld(k, 3, 0);
    uint32_t b0 = bb * cols + h * hd, i0 = b0 + 2 * m, i1 = i0 + 1;
    float a0 = ld(k, 0, i0), a1 = ld(k, 0, i1);
    st(k, 5, i0, (a0 * cc) - (a1 * ss));
    st(k, 5, i1, (a0 * ss) + (a1 * cc));
  }
}
/* rope-apply, kernels.el:1288-1304 */
static void kn_rope_apply(const K *k, uint32_t idx) {
  uint32_t seq = P(0), dim = P(1), heads = P(2);
  uint32_t hd = udiv(dim, heads), half = udiv(hd, 2);
  if (idx < (seq * heads) * half) {
    uint32_t m = umod(idx, half), tmp = udiv(idx, half);
    uint32_t h = umod(tmp, heads), p = udiv(tmp, heads);
    uint32_t ci = p * half + m;
    float cc = ld(k, 1, ci), ss = ld(k, 2, ci) * ld(k, 3, 0);
    uint32_t b0 = p * dim + h * hd, i0 = b0 + 2 * m, i1 = i0 + 1;
    float a0 = ld(k, 0, i0), a1 = ld(k, 0, i1);
    st(k, 4, i0, (a0 * cc) - (a1 * ss));
    st(k, 4, i1, (a0 * ss) + (a1 * cc));
  }
}
/* rope-half, kernels.el:844-882 (rbase and sgn arrive as f32 bit patterns) */
static void kn_rope_half(const K *k, uint32_t idx) {
  uint32_t seq = P(0), nheads = P(1), hd = P(2);
  float rbase = bits2f(P(3)), sgn = bits2f(P(4));
  uint32_t half = udiv(hd, 2);
  if (idx < (seq * nheads) * half) {
    uint32_t m = umod(idx, half), tmp = udiv(idx, half);
    uint32_t h = umod(tmp, nheads), p = udiv(tmp, nheads);
    uint32_t b0 = p * (nheads * hd) + h * hd;
    float ex = (2.0f * (float)m) / (float)hd;
    float theta = (float)p / powf(rbase, ex);
    float c = cosf(theta);
    float s = sgn * sinf(theta);
    float a0 = ld(k, 0, b0 + m), a1 = ld(k, 0, b0 + (m + half));
    st(k, 1, b0 + m, (a0 * c) - (a1 * s));
    st(k, 1, b0 + (m + half), (a1 * c) + (a0 * s));
  }
}

/* ---- row reductions --------------------------------------------------- */

/* softmax, kernels.el:28-42 */
static void kn_softmax(const K *k, uint32_t idx) {
  uint32_t M = P(0), N = P(1);
  if (idx < M) {
    uint32_t base = idx * N;
    float m = ld(k, 0, base);
    for (uint32_t j = 0; j < N; j++) {
      float v = ld(k, 0, base + j);
      if (v > m) m = v;
    }
    float s = 0.0f;
    for (uint32_t j2 = 0; j2 < N; j2++) s = s + expf(ld(k, 0, base + j2) - m);
    for (uint32_t j3 = 0; j3 < N; j3++) st(k, 1, base + j3, expf(ld(k, 0, base + j3) - m) / s);
  }
}
/* rmsnorm-istd, kernels.el:1249-1256 */
static void kn_rmsnorm_istd(const K *k, uint32_t r) {
  uint32_t M = P(0), N = P(1);
  if (r < M) {
    uint32_t base = r * N;
    float ss = 0.0f;
    for (uint32_t kk = 0; kk < N; kk++) {
      float v = ld(k, 0, base + kk);
      ss = ss + v * v;
    }
    st(k, 1, r, 1.0f / sqrtf(ss / (float)N + EPS6));
  }
}
/* rmsnorm-heads, kernels.el:823-842 */
static void kn_rmsnorm_heads(const K *k, uint32_t idx) {
  uint32_t seq = P(0), nheads = P(1), hd = P(2);
  if (idx < seq * nheads) {
    uint32_t base = idx * hd;
    float ss = 0.0f;
    for (uint32_t i = 0; i < hd; i++) {
      float v = ld(k, 0, base + i);
      ss = ss + v * v;
    }
    float inv = 1.0f / sqrtf(ss / (float)hd + EPS6);
    for (uint32_t j = 0; j < hd; j++) st(k, 2, base + j, (ld(k, 0, base + j) * inv) * ld(k, 1, j));
  }
}
/* One element of pack-act-rows / quant-act's rounding: returns ri (0..127)
 * and sets *neg; kernels.el:912-926 and :538-546. */
static inline uint32_t quant_lane(float v, float gamma, int *neg) {
  float q = 0.0f;
  if (gamma > 0.0f) q = v / gamma;
  float aq = q;
  *neg = 0;
  if (q < 0.0f) { *neg = 1; aq = 0.0f - q; }
  uint32_t ri = f2u(aq + 0.5f);
  if (ri > 127u) ri = 127u;
  return ri;
}
/* pack-act-rows, kernels.el:884-932 */
static void kn_pack_act_rows(const K *k, uint32_t row) {
  uint32_t seq = P(0), cols = P(1), ng = P(2);
  if (row < seq) {
    uint32_t base = row * cols;
    float amax = 0.0f;
    for (uint32_t c = 0; c < cols; c++) {
      float v = ld(k, 0, base + c), av = v;
      if (v < 0.0f) av = 0.0f - v;
      if (av > amax) amax = av;
    }
    float gamma = amax / 127.0f;
    st(k, 2, row, gamma);
    uint32_t wb = row * ng;
    for (uint32_t w = 0; w < ng; w++) {
      uint32_t word = 0, sh = 1;
      for (uint32_t l = 0; l < 4; l++) {
        uint32_t c = w * 4 + l, lane = 0;
        if (c < cols) {
          float v = ld(k, 0, base + c);
          float q = 0.0f;
          if (gamma > 0.0f) q = v / gamma;
          uint32_t neg = 0;
          float aq = q;
          if (q < 0.0f) { neg = 1; aq = 0.0f - q; }
          uint32_t ri = f2u(aq + 0.5f);
          if (ri > 127u) ri = 127u;
          lane = ri;
          if (neg == 1) lane = (256u - ri) % 256u;
        }
        word = word + lane * sh;
        sh = sh * 256u;
      }
      st(k, 1, wb + w, bits2f(word));
    }
  }
}
/* quant-act, kernels.el:527-547 */
static void kn_quant_act(const K *k, uint32_t row) {
  uint32_t seq = P(0), cols = P(1);
  if (row < seq) {
    uint32_t base = row * cols;
    float amax = 0.0f;
    for (uint32_t c = 0; c < cols; c++) {
      float v = ld(k, 0, base + c), av = v;
      if (v < 0.0f) av = 0.0f - v;
      if (av > amax) amax = av;
    }
    float gamma = amax / 127.0f;
    for (uint32_t c = 0; c < cols; c++) {
      float v = ld(k, 0, base + c), xq = 0.0f;
      if (gamma > 0.0f) {
        float q = v / gamma, sgn = 1.0f, aq = q;
        if (q < 0.0f) { sgn = -1.0f; aq = 0.0f - q; }
        uint32_t ri = f2u(aq + 0.5f);
        float rf = (float)ri;
        if (rf > 127.0f) rf = 127.0f;
        xq = gamma * (sgn * rf);
      }
      st(k, 1, base + c, xq);
    }
  }
}

/* ---- int8 / ternary linears -------------------------------------------- */

/* dp4a-dot, kernels.el:587-600 */
static void kn_dp4a_dot(const K *k, uint32_t i) {
  if (i < P(0)) {
    uint32_t apk = f2u(ld(k, 0, i)) + f2u(ld(k, 1, i)) * 65536u;
    uint32_t bpk = f2u(ld(k, 2, i)) + f2u(ld(k, 3, i)) * 65536u;
    st(k, 4, i, (float)sdot4(apk, bpk));
  }
}
/* bitlinear-dp4a, kernels.el:602-617 */
static void kn_bitlinear_dp4a(const K *k, uint32_t idx) {
  uint32_t seq = P(0), out = P(1), ng = P(2);
  if (idx < seq * out) {
    uint32_t s = udiv(idx, out), o = umod(idx, out), ab = s * ng, wb = o * ng;
    int32_t acc = 0;
    for (uint32_t g = 0; g < ng; g++) {
      uint32_t apk = f2u(ld(k, 0, ab + g)) + f2u(ld(k, 1, ab + g)) * 65536u;
      uint32_t wpk = f2u(ld(k, 2, wb + g)) + f2u(ld(k, 3, wb + g)) * 65536u;
      acc = iadd(acc, sdot4(apk, wpk));
    }
    st(k, 7, idx, ld(k, 4, o) + (ld(k, 5, 0) * ld(k, 6, s)) * (float)acc);
  }
}
/* bitlinear-dp4a-1f (per_row=0, kernels.el:619-634) and
 * bitlinear-dp4a-rows (per_row=1, kernels.el:636-653) */
static void dp4a_1f(const K *k, uint32_t idx, int per_row) {
  uint32_t seq = P(0), out = P(1), ng = P(2);
  if (idx < seq * out) {
    uint32_t s = udiv(idx, out), o = umod(idx, out), ab = s * ng, wb = o * ng;
    int32_t acc = 0;
    for (uint32_t g = 0; g < ng; g++) acc = iadd(acc, sdot4(ldu(k, 0, ab + g), ldu(k, 1, wb + g)));
    st(k, 5, idx, ld(k, 2, o) + (ld(k, 3, per_row ? o : 0) * ld(k, 4, s)) * (float)acc);
  }
}
static void kn_bitlinear_dp4a_1f(const K *k, uint32_t idx) { dp4a_1f(k, idx, 0); }
static void kn_bitlinear_dp4a_rows(const K *k, uint32_t idx) { dp4a_1f(k, idx, 1); }

/* ternary-rows, kernels.el:700-746 */
static void kn_ternary_rows(const K *k, uint32_t idx) {
  uint32_t seq = P(0), out = P(1), cols = P(2), nblk = P(3), wng = P(4);
  if (idx < seq * out) {
    uint32_t s = udiv(idx, out), o = umod(idx, out), xb = s * cols, wb = o * wng;
    float acc = 0.0f;
    for (uint32_t b = 0; b < nblk; b++) {
      float bacc = 0.0f;
      for (uint32_t w = 0; w < 8; w++) {
        uint32_t wi = b * 8 + w;
        if (wi < wng) {
          uint32_t wpk = ldu(k, 1, wb + wi), sh = 30;
          for (uint32_t f = 0; f < 16; f++) {
            uint32_t i = wi * 16 + f;
            if (i < cols) {
              float sv = (float)((int32_t)(wpk << sh) >> 30);
              bacc = bacc + sv * ld(k, 0, xb + i);
            }
            sh = sh - 2;
          }
        }
      }
      acc = acc + ld(k, 3, o * nblk + b) * bacc;
    }
    st(k, 4, idx, ld(k, 2, o) + acc);
  }
}
/* bitlinear-packed (per_row=0, kernels.el:992-1016) and
 * bitlinear-packed-v (per_row=1, kernels.el:1018-1040) */
static void packed_lin(const K *k, uint32_t idx, int per_row) {
  uint32_t seq = P(0), in = P(1), out = P(2), pk = P(3), fcount = P(4);
  if (idx < seq * out) {
    uint32_t s = udiv(idx, out), o = umod(idx, out);
    float acc = ld(k, 2, o), beta = ld(k, 3, per_row ? o : 0);
    uint32_t xb = s * in, rowf = o * fcount;
    for (uint32_t f = 0; f < fcount; f++) {
      uint32_t packed = f2u(ld(k, 1, rowf + f)), i0 = f * pk;
      for (uint32_t z = 0; z < pk; z++) {
        uint32_t i = i0 + z;
        if (i < in) {
          uint32_t code = packed % 4u;
          float tern = (float)code - 1.0f;
          acc = acc + ld(k, 0, xb + i) * (beta * tern);
        }
        packed = packed / 4u;
      }
    }
    st(k, 4, idx, acc);
  }
}
static void kn_bitlinear_packed(const K *k, uint32_t idx) { packed_lin(k, idx, 0); }
static void kn_bitlinear_packed_v(const K *k, uint32_t idx) { packed_lin(k, idx, 1); }

/* ---- f32 GEMM --------------------------------------------------------- */

/* matmul, kernels.el:17-27 */
static void kn_matmul(const K *k, uint32_t idx) {
  uint32_t M = P(0), Kd = P(1), N = P(2);
  if (idx < M * N) {
    uint32_t row = udiv(idx, N), col = umod(idx, N);
    float acc = 0.0f;
    for (uint32_t kk = 0; kk < Kd; kk++) acc = acc + ld(k, 0, row * Kd + kk) * ld(k, 1, kk * N + col);
    st(k, 2, idx, acc);
  }
}
/* linear, kernels.el:71-81 */
static void kn_linear(const K *k, uint32_t idx) {
  uint32_t M = P(0), IN = P(1), OUT = P(2);
  if (idx < M * OUT) {
    uint32_t row = udiv(idx, OUT), o = umod(idx, OUT);
    float acc = ld(k, 2, o);
    for (uint32_t kk = 0; kk < IN; kk++) acc = acc + ld(k, 0, row * IN + kk) * ld(k, 1, o * IN + kk);
    st(k, 3, idx, acc);
  }
}
/* matmul-tiled, kernels.el:82-107 (local size 16x16, 256 invocations per
 * workgroup).  Each tile's 16 products are summed right-nested,
 * p0 + (p1 + (... + (p14 + p15))), and that sum is added to acc. */
static void kn_matmul_tiled(const K *k, uint32_t gid) {
  uint32_t M = P(0), Kd = P(1), N = P(2);
  uint32_t wg = gid / 256u, l = gid % 256u, lc = l % 16u, lr = l / 16u;
  uint32_t tilesx = (N + 15u) / 16u;
  uint32_t trow = udiv(wg, tilesx), tcol = umod(wg, tilesx);
  uint32_t row = trow * 16u + lr, col = tcol * 16u + lc;
  float acc = 0.0f;
  uint32_t nt = (Kd + 15u) / 16u;
  for (uint32_t tt = 0; tt < nt; tt++) {
    float pr[16];
    for (uint32_t q = 0; q < 16; q++) {
      uint32_t ak = tt * 16u + q; /* As[lr][q] was loaded by lane (lr, q) */
      float a = 0.0f, bv = 0.0f;
      if (row < M && ak < Kd) a = ld(k, 0, row * Kd + ak);
      uint32_t bk = tt * 16u + q; /* Bs[q][lc] was loaded by lane (q, lc) */
      if (bk < Kd && col < N) bv = ld(k, 1, bk * N + col);
      pr[q] = a * bv;
    }
    float inner = pr[15];
    for (int q = 14; q >= 0; q--) inner = pr[q] + inner;
    acc = acc + inner;
  }
  if (row < M && col < N) st(k, 2, row * N + col, acc);
}
/* matmul-reg, kernels.el:129 (a 4x4 register micro-tile per invocation) */
static void kn_matmul_reg(const K *k, uint32_t idx) {
  uint32_t M = P(0), Kd = P(1), N = P(2);
  uint32_t bpr = (N + 3u) / 4u;
  uint32_t brow = udiv(idx, bpr) * 4u, bcol = umod(idx, bpr) * 4u;
  if (brow < M) {
    float acc[4][4];
    memset(acc, 0, sizeof acc);
    for (uint32_t kk = 0; kk < Kd; kk++) {
      float a[4], b[4];
      for (int r = 0; r < 4; r++) a[r] = ld(k, 0, (brow + r) * Kd + kk);
      for (int c = 0; c < 4; c++) b[c] = ld(k, 1, kk * N + (bcol + c));
      for (int r = 0; r < 4; r++)
        for (int c = 0; c < 4; c++) acc[r][c] = acc[r][c] + a[r] * b[c];
    }
    for (int r = 0; r < 4; r++)
      for (int c = 0; c < 4; c++) st(k, 2, (brow + r) * N + (bcol + c), acc[r][c]);
  }
}

/* ---- attention -------------------------------------------------------- */

/* attn-scores, kernels.el:205-222 */
static void kn_attn_scores(const K *k, uint32_t idx) {
  uint32_t seq = P(0), dim = P(1), heads = P(2), kvheads = P(3);
  uint32_t hd = udiv(dim, heads), grp = udiv(heads, kvheads), kvdim = kvheads * hd;
  if (idx < (heads * seq) * seq) {
    uint32_t h = udiv(idx, seq * seq), rem = umod(idx, seq * seq);
    uint32_t i = udiv(rem, seq), j = umod(rem, seq);
    if (j > i) st(k, 2, idx, NEG_BIG);
    if (j < i + 1) {
      uint32_t kvh = udiv(h, grp), qb = i * dim + h * hd, kb = j * kvdim + kvh * hd;
      float acc = 0.0f;
      for (uint32_t t = 0; t < hd; t++) acc = acc + ld(k, 0, qb + t) * ld(k, 1, kb + t);
      st(k, 2, idx, acc * (1.0f / sqrtf((float)hd)));
    }
  }
}
/* attn-context, kernels.el:223-235 */
static void kn_attn_context(const K *k, uint32_t idx) {
  uint32_t seq = P(0), dim = P(1), heads = P(2), kvheads = P(3);
  uint32_t hd = udiv(dim, heads), grp = udiv(heads, kvheads), kvdim = kvheads * hd;
  if (idx < seq * dim) {
    uint32_t i = udiv(idx, dim), c = umod(idx, dim);
    uint32_t h = udiv(c, hd), t = umod(c, hd), kvh = udiv(h, grp);
    uint32_t pb = h * (seq * seq) + i * seq;
    float acc = 0.0f;
    for (uint32_t j = 0; j < seq; j++) acc = acc + ld(k, 0, pb + j) * ld(k, 1, j * kvdim + (kvh * hd + t));
    st(k, 2, idx, acc);
  }
}
/* decode-attn (batched=0, kernels.el:315-338) and decode-attn-b
 * (batched=1, kernels.el:366-390) */
static void decode_attn(const K *k, uint32_t idx, int batched) {
  uint32_t B = batched ? P(0) : 1u, dim = P(batched ? 1 : 0), heads = P(batched ? 2 : 1);
  uint32_t kvheads = P(batched ? 3 : 2), maxseq = batched ? P(4) : 0u;
  uint32_t hd = udiv(dim, heads), grp = udiv(heads, kvheads), kvdim = kvheads * hd;
  if (idx < B * dim) {
    uint32_t bb = udiv(idx, dim), c = umod(idx, dim);
    uint32_t h = udiv(c, hd), t = umod(c, hd), kvh = udiv(h, grp);
    uint32_t pos = f2u(ld(k, 3, 0)), len = pos + 1u;
    uint32_t cbase = (bb * maxseq) * kvdim, c0q = bb * dim + h * hd;
    float coef = 1.0f / sqrtf((float)hd), mx = NEG_BIG;
    for (uint32_t j = 0; j < len; j++) {
      uint32_t kb = cbase + (j * kvdim + kvh * hd);
      float acc = 0.0f;
      for (uint32_t tt = 0; tt < hd; tt++) acc = acc + ld(k, 0, c0q + tt) * ld(k, 1, kb + tt);
      float s = acc * coef;
      if (s > mx) mx = s;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t j = 0; j < len; j++) {
      uint32_t kb = cbase + (j * kvdim + kvh * hd);
      float acc = 0.0f;
      for (uint32_t tt = 0; tt < hd; tt++) acc = acc + ld(k, 0, c0q + tt) * ld(k, 1, kb + tt);
      float e = expf(acc * coef - mx);
      z = z + e;
      ctx = ctx + e * ld(k, 2, kb + t);
    }
    st(k, 4, idx, ctx / z);
  }
}
static void kn_decode_attn(const K *k, uint32_t idx) { decode_attn(k, idx, 0); }
static void kn_decode_attn_b(const K *k, uint32_t idx) { decode_attn(k, idx, 1); }
/* attn-causal-gqa, kernels.el:934-990 */
static void kn_attn_causal_gqa(const K *k, uint32_t idx) {
  uint32_t seq = P(0), heads = P(1), kvheads = P(2), hd = P(3);
  if (idx < heads * seq) {
    uint32_t h = udiv(idx, seq), i = umod(idx, seq);
    uint32_t qdim = heads * hd, kvdim = kvheads * hd, grp = udiv(heads, kvheads);
    uint32_t qb = i * qdim + h * hd, kc = udiv(h, grp) * hd;
    float scale = 1.0f / sqrtf((float)hd);
    uint32_t n = i + 1u;
    float mx = NEG_BIG;
    for (uint32_t j = 0; j < n; j++) {
      uint32_t kb = j * kvdim + kc;
      float acc = 0.0f;
      for (uint32_t t = 0; t < hd; t++) acc = acc + ld(k, 0, qb + t) * ld(k, 1, kb + t);
      acc = acc * scale;
      if (acc > mx) mx = acc;
    }
    float sm = 0.0f;
    for (uint32_t j = 0; j < n; j++) {
      uint32_t kb = j * kvdim + kc;
      float acc = 0.0f;
      for (uint32_t t = 0; t < hd; t++) acc = acc + ld(k, 0, qb + t) * ld(k, 1, kb + t);
      sm = sm + expf(acc * scale - mx);
    }
    for (uint32_t t = 0; t < hd; t++) st(k, 3, qb + t, 0.0f);
    for (uint32_t j = 0; j < n; j++) {
      uint32_t kb = j * kvdim + kc;
      float acc = 0.0f;
      for (uint32_t t = 0; t < hd; t++) acc = acc + ld(k, 0, qb + t) * ld(k, 1, kb + t);
      float pj = expf(acc * scale - mx) / sm;
      for (uint32_t t = 0; t < hd; t++) st(k, 3, qb + t, ld(k, 3, qb + t) + pj * ld(k, 2, kb + t));
    }
  }
}

/* ---- transposed linears ------------------------------------------------ */

/* ternary-rows-t, kernels.el:748-775: WP BETA G X; push (out cols nblk wng seq) */
static void kn_ternary_rows_t(const K *k, uint32_t idx) {
  uint32_t out = P(0), cols = P(1), nblk = P(2), wng = P(3), seq = P(4);
  if (idx < seq * cols) {
    uint32_t p = udiv(idx, cols), i = umod(idx, cols);
    uint32_t b = i / 128u, wi = i / 16u, fd = i % 16u;
    uint32_t sh = 30u - 2u * fd, gb = p * out;
    float acc = 0.0f;
    for (uint32_t o = 0; o < out; o++) {
      uint32_t wpk = ldu(k, 0, o * wng + wi);
      float sv = (float)((int32_t)(wpk << sh) >> 30);
      acc = acc + sv * (ld(k, 1, o * nblk + b) * ld(k, 2, gb + o));
    }
    st(k, 3, idx, acc);
  }
}
/* dp4a-rows-t, kernels.el:777-810: WP BETA G X; push (out cols ng seq) */
static void kn_dp4a_rows_t(const K *k, uint32_t idx) {
  uint32_t out = P(0), cols = P(1), ng = P(2), seq = P(3);
  if (idx < seq * cols) {
    uint32_t p = udiv(idx, cols), i = umod(idx, cols);
    uint32_t word = i / 4u, lane = i % 4u, sh = 1u;
    for (uint32_t l = 0; l < lane; l++) sh = sh * 256u;
    uint32_t gb = p * out;
    float acc = 0.0f;
    for (uint32_t o = 0; o < out; o++) {
      uint32_t wpk = ldu(k, 0, o * ng + word);
      uint32_t b = (wpk / sh) % 256u;
      float sv = (float)((b + 128u) % 256u) - 128.0f;
      acc = acc + sv * (ld(k, 1, o) * ld(k, 2, gb + o));
    }
    st(k, 3, idx, acc);
  }
}

/* ---- long-context decode ---------------------------------------------- */

/* cache-append-ring, kernels.el:396-403 */
static void kn_cache_append_ring(const K *k, uint32_t idx) {
  uint32_t kvdim = P(0), nsink = P(1), win = P(2);
  if (idx < kvdim) {
    uint32_t pos = f2u(ld(k, 1, 0));
    uint32_t slot = pos;
    if (pos >= nsink) slot = nsink + umod(pos - nsink, win);
    st(k, 2, slot * kvdim + idx, ld(k, 0, idx));
  }
}
/* The q.k product of decode-attn-stream / attn-stream-entries: K row kb
 * rotated by cache-relative position crel, q by qcrel, pairs (2m, 2m+1)
 * (kernels.el:425-433, :1069-1077). */
static float stream_dot(const K *k, uint32_t kb, uint32_t crel, uint32_t qcrel, uint32_t c0q, uint32_t half) {
  float acc = 0.0f;
  for (uint32_t m = 0; m < half; m++) {
    uint32_t ci = crel * half + m;
    float cc = ld(k, 4, ci), ss = ld(k, 5, ci);
    float k0 = ld(k, 1, kb + 2 * m), k1 = ld(k, 1, kb + (2 * m + 1));
    float kr0 = (k0 * cc) - (k1 * ss), kr1 = (k0 * ss) + (k1 * cc);
    uint32_t qci = qcrel * half + m;
    float qcc = ld(k, 4, qci), qss = ld(k, 5, qci);
    float q0 = ld(k, 0, c0q + 2 * m), q1 = ld(k, 0, c0q + (2 * m + 1));
    float qr0 = (q0 * qcc) - (q1 * qss), qr1 = (q0 * qss) + (q1 * qcc);
    acc = acc + ((qr0 * kr0) + (qr1 * kr1));
  }
  return acc;
}
/* decode-attn-stream, kernels.el:404-451: Q CK CV POS CO SI C; push (dim heads kvheads nsink win) */
static void kn_decode_attn_stream(const K *k, uint32_t idx) {
  uint32_t dim = P(0), heads = P(1), kvheads = P(2), nsink = P(3), win = P(4);
  uint32_t hd = udiv(dim, heads), grp = udiv(heads, kvheads), kvdim = kvheads * hd, half = udiv(hd, 2);
  if (idx < dim) {
    uint32_t h = udiv(idx, hd), t = umod(idx, hd), kvh = udiv(h, grp);
    uint32_t pos = f2u(ld(k, 3, 0)), cap = nsink + win;
    uint32_t len = pos + 1;
    if (len > cap) len = cap;
    uint32_t start = nsink;
    if (pos >= cap) start = (pos - win) + 1;
    uint32_t woff = umod(start - nsink, win);
    uint32_t qcrel = pos;
    if (qcrel >= cap) qcrel = cap - 1;
    uint32_t c0q = h * hd;
    float coef = 1.0f / sqrtf((float)hd), mx = NEG_BIG;
    for (uint32_t r = 0; r < len; r++) {
      uint32_t slot = r;
      if (r >= nsink) slot = nsink + umod(woff + (r - nsink), win);
      uint32_t kb = slot * kvdim + kvh * hd;
      float s = stream_dot(k, kb, r, qcrel, c0q, half) * coef;
      if (s > mx) mx = s;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t r = 0; r < len; r++) {
      uint32_t slot = r;
      if (r >= nsink) slot = nsink + umod(woff + (r - nsink), win);
      uint32_t kb = slot * kvdim + kvh * hd;
      float e = expf(stream_dot(k, kb, r, qcrel, c0q, half) * coef - mx);
      z = z + e;
      ctx = ctx + e * ld(k, 2, slot * kvdim + (kvh * hd + t));
    }
    st(k, 6, idx, ctx / z);
  }
}
/* attn-stream-entries, kernels.el:1050-1090: Q CK CV ENT CO SI C; push (dim heads kvheads ne qcrel) */
static void kn_attn_stream_entries(const K *k, uint32_t idx) {
  uint32_t dim = P(0), heads = P(1), kvheads = P(2), ne = P(3), qcrel = P(4);
  uint32_t hd = udiv(dim, heads), grp = udiv(heads, kvheads), half = udiv(hd, 2);
  if (idx < dim) {
    uint32_t h = udiv(idx, hd), t = umod(idx, hd), kvh = udiv(h, grp);
    uint32_t c0q = h * hd;
    float coef = 1.0f / sqrtf((float)hd), mx = NEG_BIG;
    for (uint32_t r = 0; r < ne; r++) {
      uint32_t base = f2u(ld(k, 3, 2 * r)), crel = f2u(ld(k, 3, 2 * r + 1));
      float s = stream_dot(k, base + kvh * hd, crel, qcrel, c0q, half) * coef;
      if (s > mx) mx = s;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t r = 0; r < ne; r++) {
      uint32_t base = f2u(ld(k, 3, 2 * r)), crel = f2u(ld(k, 3, 2 * r + 1));
      float e = expf(stream_dot(k, base + kvh * hd, crel, qcrel, c0q, half) * coef - mx);
      z = z + e;
      ctx = ctx + e * ld(k, 2, base + (kvh * hd + t));
    }
    st(k, 6, idx, ctx / z);
  }
}
/* cache-append-paged, kernels.el:1099-1108 (per_seq 0, position POS[0]) and
 * cache-append-paged-v, :1211-1220 (per_seq 1, position LENS[s]) */
static void cache_append_paged(const K *k, uint32_t idx, int per_seq) {
  uint32_t B = P(0), kvdim = P(1), bs = P(2), mbps = P(3);
  if (idx < B * kvdim) {
    uint32_t s = udiv(idx, kvdim), t = umod(idx, kvdim);
    uint32_t pos = f2u(ld(k, 1, per_seq ? s : 0u));
    uint32_t lb = udiv(pos, bs), off = umod(pos, bs);
    uint32_t phys = f2u(ld(k, 2, s * mbps + lb));
    st(k, 3, (phys * bs + off) * kvdim + t, ld(k, 0, idx));
  }
}
static void kn_cache_append_paged(const K *k, uint32_t idx) { cache_append_paged(k, idx, 0); }
static void kn_cache_append_paged_v(const K *k, uint32_t idx) { cache_append_paged(k, idx, 1); }
/* decode-attn-paged, kernels.el:1110-1136 (per_seq 0) and decode-attn-paged-v,
 * :1222-1246 (per_seq 1): Q CK CV POS|LENS TABLE C; push (B dim heads kvheads bs mbps) */
static void decode_attn_paged(const K *k, uint32_t idx, int per_seq) {
  uint32_t B = P(0), dim = P(1), heads = P(2), kvheads = P(3), bs = P(4), mbps = P(5);
  uint32_t hd = udiv(dim, heads), grp = udiv(heads, kvheads), kvdim = kvheads * hd;
  if (idx < B * dim) {
    uint32_t s = udiv(idx, dim), c = umod(idx, dim);
    uint32_t h = udiv(c, hd), t = umod(c, hd), kvh = udiv(h, grp);
    uint32_t pos = f2u(ld(k, 3, per_seq ? s : 0u)), len = pos + 1;
    uint32_t c0q = s * dim + h * hd;
    float coef = 1.0f / sqrtf((float)hd), mx = NEG_BIG;
    for (uint32_t j = 0; j < len; j++) {
      uint32_t lb = udiv(j, bs), off = umod(j, bs);
      uint32_t phys = f2u(ld(k, 4, s * mbps + lb));
      uint32_t kb = (phys * bs + off) * kvdim + kvh * hd;
      float acc = 0.0f;
      for (uint32_t tt = 0; tt < hd; tt++) acc = acc + ld(k, 0, c0q + tt) * ld(k, 1, kb + tt);
      float sc = acc * coef;
      if (sc > mx) mx = sc;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t j = 0; j < len; j++) {
      uint32_t lb = udiv(j, bs), off = umod(j, bs);
      uint32_t phys = f2u(ld(k, 4, s * mbps + lb));
      uint32_t kb = (phys * bs + off) * kvdim + kvh * hd;
      float acc = 0.0f;
      for (uint32_t tt = 0; tt < hd; tt++) acc = acc + ld(k, 0, c0q + tt) * ld(k, 1, kb + tt);
      float e = expf(acc * coef - mx);
      z = z + e;
      ctx = ctx + e * ld(k, 2, kb + t);
    }
    st(k, 5, idx, ctx / z);
  }
}
static void kn_decode_attn_paged(const K *k, uint32_t idx) { decode_attn_paged(k, idx, 0); }
static void kn_decode_attn_paged_v(const K *k, uint32_t idx) { decode_attn_paged(k, idx, 1); }
/* block-copy, kernels.el:1182-1189: POOL; push (bs kvdim src dst) */
static void kn_block_copy(const K *k, uint32_t i) {
  uint32_t bs = P(0), kvdim = P(1), src = P(2), dst = P(3), bn = bs * kvdim;
  if (i < bn) st(k, 0, dst * bn + i, ld(k, 0, src * bn + i));
}
/* decode-rope-b-v, kernels.el:1195-1209: decode-rope-b with row bb at LENS[bb] */
static void kn_decode_rope_b_v(const K *k, uint32_t idx) {
  uint32_t B = P(0), cols = P(1), heads = P(2);
  uint32_t hd = udiv(cols, heads), half = udiv(hd, 2), rh = heads * half;
  if (idx < B * rh) {
    uint32_t bb = udiv(idx, rh), rem = umod(idx, rh);
    uint32_t m = umod(rem, half), h = udiv(rem, half);
    uint32_t pos = f2u(ld(k, 4, bb)), ci = pos * half + m;
    float cc = ld(k, 1, ci), ss = ld(k, 2, ci) * ld(k, 3, 0);
    uint32_t b0 = bb * cols + h * hd, i0 = b0 + 2 * m, i1 = i0 + 1;
    float a0 = ld(k, 0, i0), a1 = ld(k, 0, i1);
    st(k, 5, i0, (a0 * cc) - (a1 * ss));
    st(k, 5, i1, (a0 * ss) + (a1 * cc));
  }
}

/* ---- the table -------------------------------------------------------- */

typedef void (*kfn)(const K *, uint32_t);
typedef struct {
  const char *name;
  uint32_t nbuf, npush, local;
  kfn fn;
} entry;

static const entry TABLE[] = {
    {"vadd", 3, 1, 64, kn_vadd},
    {"matmul", 3, 3, 64, kn_matmul},
    {"softmax", 2, 2, 64, kn_softmax},
    {"linear", 4, 3, 64, kn_linear},
    {"matmul-tiled", 3, 3, 256, kn_matmul_tiled},
    {"matmul-reg", 3, 3, 64, kn_matmul_reg},
    {"scale", 3, 1, 64, kn_scale},
    {"causal-mask", 1, 1, 64, kn_causal_mask},
    {"silu-mul", 3, 1, 64, kn_silu_mul},
    {"attn-scores", 3, 4, 64, kn_attn_scores},
    {"attn-context", 3, 4, 64, kn_attn_context},
    {"decode-rope", 6, 2, 64, kn_decode_rope},
    {"cache-append", 3, 1, 64, kn_cache_append},
    {"decode-attn", 5, 3, 64, kn_decode_attn},
    {"decode-rope-b", 6, 3, 64, kn_decode_rope_b},
    {"cache-append-b", 3, 3, 64, kn_cache_append_b},
    {"decode-attn-b", 5, 5, 64, kn_decode_attn_b},
    {"quant-act", 2, 2, 64, kn_quant_act},
    {"dp4a-dot", 5, 1, 64, kn_dp4a_dot},
    {"bitlinear-dp4a", 8, 3, 64, kn_bitlinear_dp4a},
    {"bitlinear-dp4a-1f", 6, 3, 64, kn_bitlinear_dp4a_1f},
    {"bitlinear-dp4a-rows", 6, 3, 64, kn_bitlinear_dp4a_rows},
    {"ternary-rows", 5, 5, 64, kn_ternary_rows},
    {"add2", 3, 1, 64, kn_add2},
    {"rmsnorm-heads", 3, 3, 64, kn_rmsnorm_heads},
    {"rope-half", 2, 5, 64, kn_rope_half},
    {"pack-act-rows", 3, 3, 64, kn_pack_act_rows},
    {"attn-causal-gqa", 4, 4, 64, kn_attn_causal_gqa},
    {"bitlinear-packed", 5, 5, 64, kn_bitlinear_packed},
    {"bitlinear-packed-v", 5, 5, 64, kn_bitlinear_packed_v},
    {"qkv-append", 3, 3, 64, kn_qkv_append},
    {"rmsnorm-istd", 2, 2, 64, kn_rmsnorm_istd},
    {"rmsnorm-fwd", 4, 2, 64, kn_rmsnorm_fwd},
    {"rope-apply", 5, 3, 64, kn_rope_apply},
    {"silu", 2, 1, 64, kn_silu},
    {"mul", 3, 1, 64, kn_mul},
    {"embed-gather", 3, 2, 64, kn_embed_gather},
    {"ternary-rows-t", 4, 5, 64, kn_ternary_rows_t},
    {"dp4a-rows-t", 4, 4, 64, kn_dp4a_rows_t},
    {"cache-append-ring", 3, 3, 64, kn_cache_append_ring},
    {"decode-attn-stream", 7, 5, 64, kn_decode_attn_stream},
    {"attn-stream-entries", 7, 5, 64, kn_attn_stream_entries},
    {"cache-append-paged", 4, 4, 64, kn_cache_append_paged},
    {"decode-attn-paged", 6, 6, 64, kn_decode_attn_paged},
    {"block-copy", 1, 4, 64, kn_block_copy},
    {"decode-rope-b-v", 6, 3, 64, kn_decode_rope_b_v},
    {"cache-append-paged-v", 4, 4, 64, kn_cache_append_paged_v},
    {"decode-attn-paged-v", 6, 6, 64, kn_decode_attn_paged_v},
};
#define NTABLE ((int)(sizeof TABLE / sizeof TABLE[0]))

static const entry *find(const char *name) {
  for (int i = 0; i < NTABLE; i++)
    if (!strcmp(TABLE[i].name, name)) return &TABLE[i];
  return NULL;
}

int or_kernel_count(void) { return NTABLE; }
const char *or_kernel_name(int i) { return (i >= 0 && i < NTABLE) ? TABLE[i].name : NULL; }
int or_kernel_abi(const char *name, uint32_t *nbuf, uint32_t *npush) {
  const entry *e = find(name);
  if (!e) return 1;
  if (nbuf) *nbuf = e->nbuf;
  if (npush) *npush = e->npush;
  return 0;
}

int or_dispatch(const char *name, float **bufs, const uint32_t *sizes, uint32_t nbuf,
                const uint32_t *push, uint32_t npush, uint32_t groups) {
  const entry *e = find(name);
  if (!e || nbuf != e->nbuf || npush != e->npush) return 1;
  uint32_t zero[1] = {0};
  K k = {bufs, sizes, npush ? push : zero, 0};
  uint64_t n = (uint64_t)groups * e->local;
  if (n > 0xffffffffull) n = 0xffffffffull;
  k.nthreads = (uint32_t)n;
  /* causal-mask, attn-causal-gqa and the in-place softmax write only what
   * their own invocation reads, so invocations are independent. */
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t g = 0; g < (int64_t)n; g++) e->fn(&k, (uint32_t)g);
  return 0;
}

/* ---- typed composites ------------------------------------------------- */

void or_pack_act_rows(const float *x, uint32_t *xq, float *gamma, uint32_t seq, uint32_t cols) {
  uint32_t ng = (cols + 3u) / 4u;
  float *b[3] = {(float *)x, (float *)xq, gamma};
  uint32_t n[3] = {seq * cols, seq * ng, seq};
  uint32_t p[3] = {seq, cols, ng};
  K k = {b, n, p, seq};
#pragma omp parallel for
  for (int64_t r = 0; r < (int64_t)seq; r++) kn_pack_act_rows(&k, (uint32_t)r);
}

void or_softmax_rows(const float *a, float *c, uint32_t rows, uint32_t cols) {
  float *b[2] = {(float *)a, c};
  uint32_t n[2] = {rows * cols, rows * cols};
  uint32_t p[2] = {rows, cols};
  K k = {b, n, p, rows};
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < (int64_t)rows; r++) kn_softmax(&k, (uint32_t)r);
}

/* Unpack 2-bit word g's fields into int8-lane words: field f of word wi
 * (decoded as in ternary-rows, kernels.el:728-743) becomes lane f%4 of
 * lane-word 4*wi + f/4, so the weight row lines up with pack-act-rows'
 * activation words (4 lanes per word, lane l = column 4w+l). */
static inline uint32_t unpack_lane_word(const uint32_t *wrow, uint32_t wng, uint32_t g,
                                        uint32_t cols) {
  uint32_t wi = g / 4u, word = 0;
  uint32_t wpk = wi < wng ? wrow[wi] : 0u;
  for (uint32_t l = 0; l < 4; l++) {
    uint32_t f = (g % 4u) * 4u + l;
    uint32_t col = wi * 16u + f;
    int32_t v = (col < cols) ? ((int32_t)(wpk << (30u - 2u * f)) >> 30) : 0;
    word |= ((uint32_t)(uint8_t)(int8_t)v) << (8 * l);
  }
  return word;
}

void or_ternary_acc_i8(const uint32_t *xq, const uint32_t *w2, int32_t *acc, uint32_t seq,
                       uint32_t out, uint32_t cols) {
  uint32_t ng = (cols + 3u) / 4u, wng = (cols + 15u) / 16u;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < (int64_t)out; o++) {
    const uint32_t *wrow = w2 + (size_t)o * wng;
    for (uint32_t s = 0; s < seq; s++) {
      int32_t a = 0;
      for (uint32_t g = 0; g < ng; g++)
        a = iadd(a, sdot4(xq[(size_t)s * ng + g], unpack_lane_word(wrow, wng, g, cols)));
      acc[(size_t)s * out + o] = a;
    }
  }
}

void or_ternary_linear_i8(const uint32_t *xq, const float *gamma, const uint32_t *w2,
                          const float *bias, const float *beta, int beta_per_row, float *y,
                          uint32_t seq, uint32_t out, uint32_t cols) {
  uint32_t ng = (cols + 3u) / 4u, wng = (cols + 15u) / 16u;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < (int64_t)out; o++) {
    const uint32_t *wrow = w2 + (size_t)o * wng;
    /* the weight row unpacked once per output, reused for every token */
    for (uint32_t s = 0; s < seq; s++) {
      int32_t a = 0;
      for (uint32_t g = 0; g < ng; g++)
        a = iadd(a, sdot4(xq[(size_t)s * ng + g], unpack_lane_word(wrow, wng, g, cols)));
      float bo = bias ? bias[o] : 0.0f;
      float be = beta[beta_per_row ? o : 0];
      /* Y = BIAS[o] + (BETA * GAMMA[s]) * float(acc), kernels.el:633 */
      y[(size_t)s * out + o] = bo + (be * gamma[s]) * (float)a;
    }
  }
}

/* ---- decoder-stack pieces ---------------------------------------------- */

/* rmsnorm-istd then rmsnorm-fwd (kernels.el:1249-1265) with the epsilon a
 * parameter (the DSL kernel hard-codes 1e-6): S = 1/sqrt(ss/N + eps) with ss
 * the serial sum of x*x, C = (X*S)*G. */
void or_rmsnorm_rows(const float *x, const float *gain, float eps, float *y, uint32_t rows,
                     uint32_t cols) {
  for (uint32_t r = 0; r < rows; r++) {
    const float *xr = x + (size_t)r * cols;
    float ss = 0.0f;
    for (uint32_t k = 0; k < cols; k++) ss = ss + xr[k] * xr[k];
    float s = 1.0f / sqrtf(ss / (float)cols + eps);
    for (uint32_t j = 0; j < cols; j++) y[(size_t)r * cols + j] = (xr[j] * s) * gain[j];
  }
}

static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u, u;
  if (e == 31u) {
    u = sign | 0x7f800000u | (m << 13);
  } else if (e == 0u) {
    if (!m) {
      u = sign;
    } else { /* subnormal: m * 2^-24 exactly */
      float f = (float)m * 5.9604644775390625e-8f;
      memcpy(&u, &f, 4);
      u |= sign;
    }
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  return bits2f(u);
}

/* decode-attn-b (kernels.el:366-390) with K and V read from fp16 caches
 * laid out [B][kvheads][max_seq][hd]: per output element (b, h, t), serial
 * q.k dot, s = acc*coef, mx seeded at -1e30, e = exp(s - mx), z = sum e,
 * ctx = sum e*v, C = ctx/z, over positions 0..pos. */
void or_decode_attn_f16(const float *q, const uint16_t *kc, const uint16_t *vc, uint32_t pos,
                        float *out, uint32_t B, uint32_t heads, uint32_t kvheads, uint32_t hd,
                        uint32_t max_seq) {
  const uint32_t dim = heads * hd, grp = heads / kvheads, len = pos + 1u;
  const float coef = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < (int64_t)B * dim; idx++) {
    uint32_t bb = (uint32_t)(idx / dim), c = (uint32_t)(idx % dim);
    uint32_t h = c / hd, t = c % hd, kvh = h / grp;
    const float *qh = q + (size_t)bb * dim + (size_t)h * hd;
    size_t cb = ((size_t)bb * kvheads + kvh) * max_seq * hd;
    float mx = NEG_BIG;
    for (uint32_t j = 0; j < len; j++) {
      float acc = 0.0f;
      for (uint32_t tt = 0; tt < hd; tt++) acc = acc + qh[tt] * f16_to_f32(kc[cb + (size_t)j * hd + tt]);
      float s = acc * coef;
      if (s > mx) mx = s;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t j = 0; j < len; j++) {
      float acc = 0.0f;
      for (uint32_t tt = 0; tt < hd; tt++) acc = acc + qh[tt] * f16_to_f32(kc[cb + (size_t)j * hd + tt]);
      float e = expf(acc * coef - mx);
      z = z + e;
      ctx = ctx + e * f16_to_f32(vc[cb + (size_t)j * hd + t]);
    }
    out[idx] = ctx / z;
  }
}

int or_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
void or_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ---------------------------------------------------------- weight ingest */

/* Set column `col`'s 2-bit field in a zeroed [out x wng] buffer. */
static inline void put2(uint32_t *w2row, uint32_t col, int32_t v) {
  w2row[col / 16u] |= ((uint32_t)v & 3u) << (2u * (col % 16u));
}

/* int8 lanes -> 2-bit: column i is lane i%4 of word i/4 (kernels.el:619-653,
 * OpSDot's byte order), the field its value's low two bits when it lies in
 * [-2, 1] (the values ternary-rows' sign extension produces, kernels.el:728-743). */
uint32_t or_repack_i8_2bit(const uint32_t *wp, uint32_t out, uint32_t cols, uint32_t *w2) {
  const uint32_t ng = (cols + 3u) / 4u, wng = (cols + 15u) / 16u;
  uint32_t bad = 0;
  memset(w2, 0, (size_t)out * wng * 4);
  for (uint32_t o = 0; o < out; o++)
    for (uint32_t i = 0; i < cols; i++) {
      int32_t v = (int32_t)(int8_t)(wp[(size_t)o * ng + i / 4u] >> (8u * (i % 4u)));
      if (v < -2 || v > 1) bad++;
      else put2(w2 + (size_t)o * wng, i, v);
    }
  return bad;
}

/* base-4 codes -> 2-bit, peeling codes as bitlinear-packed does
 * (kernels.el:1002-1013: code = packed % 4, then packed = packed / 4). */
uint32_t or_repack_packed_2bit(const float *wpk, uint32_t out, uint32_t cols, uint32_t pk, uint32_t fcount,
                               uint32_t *w2) {
  const uint32_t wng = (cols + 15u) / 16u;
  uint32_t bad = 0;
  memset(w2, 0, (size_t)out * wng * 4);
  for (uint32_t o = 0; o < out; o++)
    for (uint32_t f = 0; f < fcount; f++) {
      uint32_t packed = f2u(wpk[(size_t)o * fcount + f]);
      for (uint32_t z = 0; z < pk; z++) {
        uint32_t i = f * pk + z;
        if (i < cols) {
          uint32_t code = packed % 4u;
          if (code == 3u) bad++;
          else put2(w2 + (size_t)o * wng, i, (int32_t)code - 1);
        }
        packed = packed / 4u;
      }
    }
  return bad;
}

/* decode-attn-paged-v (kernels.el:1222-1246) with K and V read from fp16
 * pools [block][bs][kvheads][hd]: sequence s attends positions 0..lens[s]
 * through table[s*mbps + j/bs] (offset j%bs); blocks outside [0, npool)
 * read as zero rows (the pools' bounds). */
void or_decode_attn_paged_f16(const float *q, const uint16_t *kp, const uint16_t *vp, const int32_t *lens,
                              const int32_t *table, uint32_t npool, float *out, uint32_t B, uint32_t heads,
                              uint32_t kvheads, uint32_t hd, uint32_t bs, uint32_t mbps) {
  const uint32_t dim = heads * hd, grp = heads / kvheads, kvdim = kvheads * hd;
  const float coef = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < (int64_t)B * dim; idx++) {
    uint32_t s = (uint32_t)(idx / dim), c = (uint32_t)(idx % dim);
    uint32_t h = c / hd, t = c % hd, kvh = h / grp;
    const float *qh = q + (size_t)s * dim + (size_t)h * hd;
    int32_t pos = lens[s];
    uint32_t len = pos < 0 ? 1u : (uint32_t)pos + 1u;
    if (len > bs * mbps) len = bs * mbps;
    float mx = NEG_BIG;
    for (uint32_t j = 0; j < len; j++) {
      int32_t ph = table[(size_t)s * mbps + j / bs];
      float acc = 0.0f;
      if (ph >= 0 && (uint32_t)ph < npool) {
        size_t kb = (((size_t)ph * bs + j % bs) * kvdim) + (size_t)kvh * hd;
        for (uint32_t tt = 0; tt < hd; tt++) acc = acc + qh[tt] * f16_to_f32(kp[kb + tt]);
      }
      float sc = acc * coef;
      if (sc > mx) mx = sc;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t j = 0; j < len; j++) {
      int32_t ph = table[(size_t)s * mbps + j / bs];
      float acc = 0.0f, v = 0.0f;
      if (ph >= 0 && (uint32_t)ph < npool) {
        size_t kb = (((size_t)ph * bs + j % bs) * kvdim) + (size_t)kvh * hd;
        for (uint32_t tt = 0; tt < hd; tt++) acc = acc + qh[tt] * f16_to_f32(kp[kb + tt]);
        v = f16_to_f32(vp[kb + t]);
      }
      float e = expf(acc * coef - mx);
      z = z + e;
      ctx = ctx + e * v;
    }
    out[idx] = ctx / z;
  }
}

/* decode-attn-stream (kernels.el:404-451) over fp16 ring caches
 * [B][kvheads][nsink + win][hd], sequence s at stream position pos[s]
 * (negative: 0): ranks r < len = min(pos + 1, cap) walk sink slots then the
 * ring from its oldest slot; K is rotated by r and q by qcrel = min(pos,
 * cap - 1) with the CO/SI tables, pairs (2m, 2m+1); per output element a
 * serial q.k, mx seeded at -1e30, e = exp(s - mx), C = sum(e*v)/sum(e). */
static float ring_dot(const float *qh, const uint16_t *kr, const float *co, const float *si, uint32_t r,
                      uint32_t qcrel, uint32_t half) {
  float acc = 0.0f;
  for (uint32_t m = 0; m < half; m++) {
    float cc = co[(size_t)r * half + m], ss = si[(size_t)r * half + m];
    float k0 = f16_to_f32(kr[2 * m]), k1 = f16_to_f32(kr[2 * m + 1]);
    float kr0 = (k0 * cc) - (k1 * ss), kr1 = (k0 * ss) + (k1 * cc);
    float qcc = co[(size_t)qcrel * half + m], qss = si[(size_t)qcrel * half + m];
    float q0 = qh[2 * m], q1 = qh[2 * m + 1];
    float qr0 = (q0 * qcc) - (q1 * qss), qr1 = (q0 * qss) + (q1 * qcc);
    acc = acc + ((qr0 * kr0) + (qr1 * kr1));
  }
  return acc;
}
void or_decode_attn_stream_f16(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos,
                               const float *co, const float *si, float *out, uint32_t B, uint32_t heads,
                               uint32_t kvheads, uint32_t hd, uint32_t nsink, uint32_t win) {
  const uint32_t dim = heads * hd, grp = heads / kvheads, half = hd / 2, cap = nsink + win;
  const float coef = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < (int64_t)B * dim; idx++) {
    uint32_t s = (uint32_t)(idx / dim), c = (uint32_t)(idx % dim);
    uint32_t h = c / hd, t = c % hd, kvh = h / grp;
    const float *qh = q + (size_t)s * dim + (size_t)h * hd;
    const uint16_t *kb = kc + ((size_t)s * kvheads + kvh) * cap * hd;
    const uint16_t *vb = vc + ((size_t)s * kvheads + kvh) * cap * hd;
    uint32_t p = pos[s] < 0 ? 0u : (uint32_t)pos[s];
    uint32_t len = p + 1 < cap ? p + 1 : cap;
    uint32_t start = nsink;
    if (p >= cap) start = (p - win) + 1;
    uint32_t woff = (start - nsink) % win, qcrel = p < cap ? p : cap - 1;
    float mx = NEG_BIG;
    for (uint32_t r = 0; r < len; r++) {
      uint32_t slot = r < nsink ? r : nsink + (woff + (r - nsink)) % win;
      float sc = ring_dot(qh, kb + (size_t)slot * hd, co, si, r, qcrel, half) * coef;
      if (sc > mx) mx = sc;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t r = 0; r < len; r++) {
      uint32_t slot = r < nsink ? r : nsink + (woff + (r - nsink)) % win;
      float e = expf(ring_dot(qh, kb + (size_t)slot * hd, co, si, r, qcrel, half) * coef - mx);
      z = z + e;
      ctx = ctx + e * f16_to_f32(vb[(size_t)slot * hd + t]);
    }
    out[idx] = ctx / z;
  }
}

/* attn-stream-entries (kernels.el:1052-1090) over fp16 caches
 * [B][kvheads][nslots][hd]: sequence s attends the ne rows of its entry list
 * ent[s] = (slot, rank) pairs, K rotated by the rank and q by qrank[s], in the
 * DSL body's operation order.  A slot outside [0, nslots) reads as a zero row
 * and a rank outside [0, trows) as a zero rotation (robust buffer access). */
static float ent_dot(const float *qh, const uint16_t *kr, const float *co, const float *si, int32_t rank,
                     int32_t qrank, uint32_t trows, uint32_t half) {
  float acc = 0.0f;
  int rok = rank >= 0 && (uint32_t)rank < trows, qok = qrank >= 0 && (uint32_t)qrank < trows;
  for (uint32_t m = 0; m < half; m++) {
    float cc = rok ? co[(size_t)rank * half + m] : 0.0f, ss = rok ? si[(size_t)rank * half + m] : 0.0f;
    float k0 = kr ? f16_to_f32(kr[2 * m]) : 0.0f, k1 = kr ? f16_to_f32(kr[2 * m + 1]) : 0.0f;
    float kr0 = (k0 * cc) - (k1 * ss), kr1 = (k0 * ss) + (k1 * cc);
    float qcc = qok ? co[(size_t)qrank * half + m] : 0.0f, qss = qok ? si[(size_t)qrank * half + m] : 0.0f;
    float q0 = qh[2 * m], q1 = qh[2 * m + 1];
    float qr0 = (q0 * qcc) - (q1 * qss), qr1 = (q0 * qss) + (q1 * qcc);
    acc = acc + ((qr0 * kr0) + (qr1 * kr1));
  }
  return acc;
}
void or_attn_entries_f16(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *ent,
                         const int32_t *qrank, const float *co, const float *si, float *out, uint32_t B,
                         uint32_t heads, uint32_t kvheads, uint32_t hd, uint32_t nslots, uint32_t ne,
                         uint32_t trows) {
  const uint32_t dim = heads * hd, grp = heads / kvheads, half = hd / 2;
  const float coef = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < (int64_t)B * dim; idx++) {
    uint32_t s = (uint32_t)(idx / dim), c = (uint32_t)(idx % dim);
    uint32_t h = c / hd, t = c % hd, kvh = h / grp;
    const float *qh = q + (size_t)s * dim + (size_t)h * hd;
    const uint16_t *kb = kc + ((size_t)s * kvheads + kvh) * nslots * hd;
    const uint16_t *vb = vc + ((size_t)s * kvheads + kvh) * nslots * hd;
    const int32_t *es = ent + (size_t)s * ne * 2;
    float mx = NEG_BIG;
    for (uint32_t r = 0; r < ne; r++) {
      int32_t sl = es[2 * r];
      const uint16_t *kr = sl >= 0 && (uint32_t)sl < nslots ? kb + (size_t)sl * hd : NULL;
      float sc = ent_dot(qh, kr, co, si, es[2 * r + 1], qrank[s], trows, half) * coef;
      if (sc > mx) mx = sc;
    }
    float z = 0.0f, ctx = 0.0f;
    for (uint32_t r = 0; r < ne; r++) {
      int32_t sl = es[2 * r];
      int ok = sl >= 0 && (uint32_t)sl < nslots;
      const uint16_t *kr = ok ? kb + (size_t)sl * hd : NULL;
      float e = expf(ent_dot(qh, kr, co, si, es[2 * r + 1], qrank[s], trows, half) * coef - mx);
      z = z + e;
      ctx = ctx + e * (ok ? f16_to_f32(vb[(size_t)sl * hd + t]) : 0.0f);
    }
    out[idx] = ctx / z;
  }
}
