// nlg_quant.h -- device helpers shared by the ternary kernels: the exact
// int8 activation rounding of pack-act-rows and the 2-bit x int8 dot.
#pragma once

#include "nlg_internal.h"

// ------------------------------------------------------------ quantisation

// |v| as the DSL computes it: (when (< v 0.0) (set av (- 0.0 v))).
__device__ __forceinline__ float dsl_abs(float v) { return v < 0.0f ? 0.0f - v : v; }

// One lane of pack-act-rows (kernels.el:912-926): returns the stored byte.
__device__ __forceinline__ uint32_t pack_lane(float v, float gamma) {
  float q = 0.0f;
  if (gamma > 0.0f) q = v / gamma;
  uint32_t neg = 0;
  float aq = q;
  if (q < 0.0f) {
    neg = 1;
    aq = 0.0f - q;
  }
  uint32_t ri = nlg_f2u(aq + 0.5f);
  if (ri > 127u) ri = 127u;
  return neg ? (256u - ri) % 256u : ri;
}

// ---- exact quantisation without a division per element ----
//
// pack-act-rows' lane is ri = min(trunc(RN(|q| + 0.5)), 127) with
// q = RN(v/gamma), stored as the low byte of ri, or of -ri when q < 0.
// The quotient comes from the row's reciprocal y = RN(1/gamma) (one IEEE
// division per row) and one correction step (Markstein): q0 = RN(v*y),
// r = v - q0*gamma (exact in one fma), q = RN(q0 + r*y) (one fma).  With y
// correctly rounded, q0 within an ulp of v/gamma and no underflow, q is
// exactly the correctly rounded quotient RN(v/gamma) -- the reference's
// OpFDiv result under IEEE rounding -- for every v (pinned on the CPU across
// every rounding boundary of many scales in tests/test_quant_rule.py).
// gamma >= 2^-90 keeps the remainder clear of underflow; rows with a smaller
// (or zero, or infinite) gamma divide per element (`fast` false).
// RN is symmetric, so RN(|q| + 0.5) with q's sign is RN(q + copysign(0.5, v))
// (q has v's sign, -0 included), and its truncation is +-ri.  NaN converts
// to 0, the reference's (uint f) of NaN.  Seven instructions per lane, no
// branch: mul, two fma, copysign, add, convert, clamp (the clamp never binds
// when gamma comes from the row's own absmax: |q| <= 127.0000077), plus a
// quarter of a byte pack.  (The previous estimate-and-fix-up form spent
// ~0.5 us of a 4096-column decode GEMV in its fix-up branches.)
__device__ __forceinline__ bool quant_fast(float gamma) { return gamma >= 0x1p-90f && gamma < INFINITY; }
__device__ __forceinline__ int32_t lane_q8(float v, float gamma, float ginv) {
  const float q0 = v * ginv;
  const float q = fmaf(fmaf(-q0, gamma, v), ginv, q0);  // RN(v / gamma)
  const float s = q + __builtin_copysignf(0.5f, v);
  int32_t t;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(t) : "v"(s));  // truncates; NaN -> 0 (no poison)
  return min(max(t, -127), 127);
}
// pack-act-rows' gamma = RN(amax / 127): the same correction step with the
// constant RN(1/127) (amax >= 2^-90, so nothing underflows; smaller, zero,
// infinite or NaN amax take the IEEE division) -- three instructions in
// place of the division's dozen on the path every workgroup waits on.
__device__ __forceinline__ float nlg_gamma_of(float amax) {
  if (__builtin_expect(!(amax >= 0x1p-90f && amax < INFINITY), 0)) return amax / 127.0f;
  const float y = 0.007874015718698501587f;  // RN(1/127)
  const float q0 = amax * y;
  return fmaf(fmaf(-q0, 127.0f, amax), y, q0);
}
// the low bytes of a, b, c, d as one word (a in bits 0..7)
__device__ __forceinline__ uint32_t pack_low_bytes(int32_t a, int32_t b, int32_t c, int32_t d) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
  return lo | hi;
}
// The packed word pack-act-rows stores for v.  `fast` (quant_fast(gamma))
// is uniform across the block.
__device__ __forceinline__ uint32_t quant_word(float4 v, float gamma, float ginv, bool fast) {
  if (__builtin_expect(!fast, 0))
    return pack_lane(v.x, gamma) | (pack_lane(v.y, gamma) << 8) | (pack_lane(v.z, gamma) << 16) |
           (pack_lane(v.w, gamma) << 24);
  return pack_low_bytes(lane_q8(v.x, gamma, ginv), lane_q8(v.y, gamma, ginv), lane_q8(v.z, gamma, ginv),
                        lane_q8(v.w, gamma, ginv));
}

// All N words a thread quantises, behind one uniform branch: with the test
// per word, the compiler could not interleave the words' dependent chains
// (and re-tested `fast` around each), 0.2 us of a 4096^2 decode GEMV.
template <int N>
__device__ __forceinline__ void quant_words(const float4 (&v)[N], float gamma, float ginv, bool fast,
                                            uint32_t (&w)[N]) {
  if (__builtin_expect(fast, 1)) {
#pragma unroll
    for (int k = 0; k < N; k++)
      w[k] = pack_low_bytes(lane_q8(v[k].x, gamma, ginv), lane_q8(v[k].y, gamma, ginv),
                            lane_q8(v[k].z, gamma, ginv), lane_q8(v[k].w, gamma, ginv));
  } else {
#pragma unroll
    for (int k = 0; k < N; k++)
      w[k] = pack_lane(v[k].x, gamma) | (pack_lane(v[k].y, gamma) << 8) | (pack_lane(v[k].z, gamma) << 16) |
             (pack_lane(v[k].w, gamma) << 24);
  }
}

// 4x4 byte transpose: X[k] holds columns 4k..4k+3 of a 16-column group;
// Y[s] byte k = X[k] byte s = column 4k+s, the order the masked weight
// bytes of field group s come in.
__device__ __forceinline__ void xpose4(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                       uint32_t &y0, uint32_t &y1, uint32_t &y2, uint32_t &y3) {
  const uint32_t a = __builtin_amdgcn_perm(x1, x0, 0x05010400u);  // x0.b0 x1.b0 x0.b1 x1.b1
  const uint32_t b = __builtin_amdgcn_perm(x1, x0, 0x07030602u);  // x0.b2 x1.b2 x0.b3 x1.b3
  const uint32_t c = __builtin_amdgcn_perm(x3, x2, 0x05010400u);  // x2.b0 x3.b0 x2.b1 x3.b1
  const uint32_t d = __builtin_amdgcn_perm(x3, x2, 0x07030602u);  // x2.b2 x3.b2 x2.b3 x3.b3
  y0 = __builtin_amdgcn_perm(c, a, 0x05040100u);
  y1 = __builtin_amdgcn_perm(c, a, 0x07060302u);
  y2 = __builtin_amdgcn_perm(d, b, 0x05040100u);
  y3 = __builtin_amdgcn_perm(d, b, 0x07060302u);
}

// 64 x (sum over the 16 fields of w of decode(field) * x[column]).
__device__ __forceinline__ int wdot(uint32_t w, uint32_t y0, uint32_t y1, uint32_t y2, uint32_t y3,
                                    int acc) {
  acc = __builtin_amdgcn_sdot4((int)((w << 6) & 0xC0C0C0C0u), (int)y0, acc, false);
  acc = __builtin_amdgcn_sdot4((int)((w << 4) & 0xC0C0C0C0u), (int)y1, acc, false);
  acc = __builtin_amdgcn_sdot4((int)((w << 2) & 0xC0C0C0C0u), (int)y2, acc, false);
  acc = __builtin_amdgcn_sdot4((int)(w & 0xC0C0C0C0u), (int)y3, acc, false);
  return acc;
}
