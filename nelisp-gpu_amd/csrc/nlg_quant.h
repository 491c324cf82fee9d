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
// pack-act-rows' lane magnitude is ri = min(trunc(t'), 127) with
// t' = RN(RN(|v|/gamma) + 0.5).  With ginv = RN(1/gamma) finite, the estimate
// t = RN(|v|*ginv + 0.5) (one fused rounding) differs from t' by less than
// 3e-5 whenever t < 128 (the reciprocal errs by at most 2^-24 relative on a
// quotient below 128.5, and each of the three roundings by half an ulp of a
// value below 128.5), so trunc(t) == trunc(t') unless t lies within 2^-13 of
// an integer, i.e. unless |frac(t) - 1/2| > 1/2 - 2^-13 (both sides exact).
// t >= 128 means t' > 127.99, which the clamp maps to 127 either way.  The
// few elements inside that band (and NaNs) are recomputed with the
// reference's IEEE division.  |v|/gamma = |v/gamma| under round-to-nearest,
// and a nonzero lane implies |v/gamma| >= 0.5, so the sign is v's: the
// stored byte is the low byte of the signed magnitude, (256 - ri) % 256 for
// a negative v.  About 9 instructions per lane: fma, trunc, two subtracts, a
// compare, min, copysign, convert and a third of a byte permute.
__device__ __forceinline__ int32_t lane_est(float v, float ginv, bool &near) {
  const float t = fmaf(fabsf(v), ginv, 0.5f);
  const float kf = truncf(t);
  near = !(fabsf((t - kf) - 0.5f) <= 0.5f - 0x1p-13f);  // NaN lands here
  return (int32_t)__builtin_copysignf(fminf(kf, 127.0f), v);
}
// the low bytes of a, b, c, d as one word (a in bits 0..7)
__device__ __forceinline__ uint32_t pack_low_bytes(int32_t a, int32_t b, int32_t c, int32_t d) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
  return lo | hi;
}
// The packed word pack-act-rows stores for v.  `fast` (1/gamma finite and
// gamma > 0) is uniform across the block.  The exact fix-up of flagged lanes
// sits behind a wave-uniform vote, so a wave with no flagged lane skips it.
__device__ __forceinline__ uint32_t quant_word(float4 v, float gamma, float ginv, bool fast) {
  if (!fast)
    return pack_lane(v.x, gamma) | (pack_lane(v.y, gamma) << 8) | (pack_lane(v.z, gamma) << 16) |
           (pack_lane(v.w, gamma) << 24);
  bool n0, n1, n2, n3;
  const int32_t k0 = lane_est(v.x, ginv, n0), k1 = lane_est(v.y, ginv, n1);
  const int32_t k2 = lane_est(v.z, ginv, n2), k3 = lane_est(v.w, ginv, n3);
  uint32_t w = pack_low_bytes(k0, k1, k2, k3);
  if (__builtin_amdgcn_ballot_w64(n0 || n1 || n2 || n3) != 0ull) {
    if (n0) w = (w & 0xFFFFFF00u) | pack_lane(v.x, gamma);
    if (n1) w = (w & 0xFFFF00FFu) | (pack_lane(v.y, gamma) << 8);
    if (n2) w = (w & 0xFF00FFFFu) | (pack_lane(v.z, gamma) << 16);
    if (n3) w = (w & 0x00FFFFFFu) | (pack_lane(v.w, gamma) << 24);
  }
  return w;
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
