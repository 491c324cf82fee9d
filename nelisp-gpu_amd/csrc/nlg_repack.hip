// Weight ingest: the reference's two other ternary weight formats repacked
// into the 2-bit layout every ternary entry point here reads.
//
//   int8 lanes   bitlinear-dp4a-1f / -rows (kernels.el:619-653): WP[out x ng]
//                u32 words, ng = ceil(cols/4), lane l of word g (bits 8l..8l+7,
//                a signed byte) is column 4g + l.
//   base-4       bitlinear-packed / -v (kernels.el:992-1040): WPK[out x fcount]
//                f32 values read with (uint f); column f*pk + z holds the code
//                (packed / 4^z) % 4 and the weight is code - 1; columns past
//                fcount*pk carry no weight.
//   2-bit        ternary-rows (kernels.el:700-746): W2[out x wng] u32 words,
//                wng = ceil(cols/16), field f of word w (bits 2f..2f+1) is
//                column 16w + f, decoded by sign extension (00 0, 01 +1,
//                11 -1, 10 -2); fields past cols are 0.
//
// One thread per 2-bit word.  A weight the 2-bit code cannot hold (an int8
// lane outside [-2, 1], base-4 code 3) is written as 0 and counted.

#include "nlg_internal.h"

namespace {

__device__ __forceinline__ uint32_t code2(int32_t v) { return (uint32_t)v & 3u; }

// VEC: rows are a whole number of 16-byte groups (ng % 4 == 0), so a thread's
// four lane words are one aligned 16-byte load.
template <bool VEC>
__global__ __launch_bounds__(256) void k_repack_i8(const uint32_t *wp, uint32_t out, uint32_t cols, uint32_t ng,
                                                   uint32_t wng, uint32_t *w2, uint32_t *nbad) {
  const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (uint64_t)out * wng) return;
  const uint32_t o = (uint32_t)(idx / wng), wi = (uint32_t)(idx % wng);
  const uint32_t *row = wp + (size_t)o * ng;
  uint32_t lw[4];
  if (VEC) {
    const uint4 u = nlg_ld_stream((const uint4 *)(row + 4 * wi));  // read once, written once
    lw[0] = u.x; lw[1] = u.y; lw[2] = u.z; lw[3] = u.w;
  } else {
#pragma unroll
    for (int k = 0; k < 4; k++) lw[k] = 4 * wi + k < ng ? row[4 * wi + k] : 0u;
  }
  uint32_t word = 0, bad = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t lanes = lw[k];
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t f = 4 * k + l, col = 16 * wi + f;
      const int32_t v = (int32_t)(int8_t)(lanes >> (8 * l));
      const bool ok = v >= -2 && v <= 1;
      if (col < cols) {
        if (ok) word |= code2(v) << (2 * f);
        else bad++;
      }
    }
  }
  __builtin_nontemporal_store(word, &w2[idx]);
  if (nbad && bad) atomicAdd(nbad, bad);
}

// A word's 16 columns span at most NF consecutive floats (NF = 16 when
// pk = 1, 5 once pk >= 4): all are loaded up front (clamped to the row), then
// the codes are read as (packed >> 2z) & 3, which is what z divisions by 4
// and a % 4 leave of a uint.
template <int NF>
__global__ __launch_bounds__(256) void k_repack_packed(const float *wpk, uint32_t out, uint32_t cols, uint32_t pk,
                                                       uint32_t fcount, uint32_t wng, uint32_t *w2, uint32_t *nbad) {
  const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (uint64_t)out * wng) return;
  const uint32_t o = (uint32_t)(idx / wng), wi = (uint32_t)(idx % wng);
  const float *row = wpk + (size_t)o * fcount;
  const uint32_t f0 = 16 * wi / pk;
  uint32_t pv[NF];
#pragma unroll
  for (int j = 0; j < NF; j++) {
    const uint32_t fi = f0 + j < fcount ? f0 + j : fcount - 1;
    pv[j] = nlg_f2u(row[fi]);
  }
  uint32_t word = 0, bad = 0, z = 16 * wi - f0 * pk, j = 0;
#pragma unroll
  for (int f = 0; f < 16; f++) {
    const uint32_t col = 16 * wi + f, fi = f0 + j;
    if (col < cols && fi < fcount) {
      uint32_t packed = pv[0];
#pragma unroll
      for (int k = 1; k < NF; k++) packed = j == (uint32_t)k ? pv[k] : packed;
      const uint32_t code = (packed >> (2 * z)) & 3u;
      if (code == 3u) bad++;
      else word |= code2((int32_t)code - 1) << (2 * f);
    }
    if (++z == pk) { z = 0; j++; }
  }
  w2[idx] = word;
  if (nbad && bad) atomicAdd(nbad, bad);
}

}  // namespace

extern "C" int nlg_repack_i8_to_2bit(const uint32_t *wp, uint32_t out, uint32_t cols, uint32_t *w2,
                                     uint32_t *nbad, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!out || !cols) return NLG_OK;
  if (!wp || !w2) return nlg_fail("repack i8: null weights");
  const uint32_t ng = (cols + 3) / 4, wng = (cols + 15) / 16;
  const uint64_t n = (uint64_t)out * wng;
  const dim3 grid((unsigned)((n + 255) / 256)), blk(256);
  if (ng % 4 == 0 && ((uintptr_t)wp & 15) == 0)
    hipLaunchKernelGGL(k_repack_i8<true>, grid, blk, 0, nlg_stream(stream), wp, out, cols, ng, wng, w2, nbad);
  else
    hipLaunchKernelGGL(k_repack_i8<false>, grid, blk, 0, nlg_stream(stream), wp, out, cols, ng, wng, w2, nbad);
  NLG_LAUNCHED("repack int8 lanes to 2-bit");
  return NLG_OK;
}

extern "C" int nlg_repack_packed_to_2bit(const float *wpk, uint32_t out, uint32_t cols, uint32_t pk,
                                         uint32_t fcount, uint32_t *w2, uint32_t *nbad, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!out || !cols) return NLG_OK;
  if (!wpk || !w2) return nlg_fail("repack base-4: null weights");
  if (!pk || pk > 16) return nlg_fail("repack base-4: pk %u not in 1..16", pk);
  const uint32_t wng = (cols + 15) / 16;
  const uint64_t n = (uint64_t)out * wng;
  if (!fcount) return nlg_fail("repack base-4: fcount is 0");
  const dim3 grid((unsigned)((n + 255) / 256)), blk(256);
  if (pk >= 4)
    hipLaunchKernelGGL(k_repack_packed<5>, grid, blk, 0, nlg_stream(stream), wpk, out, cols, pk, fcount, wng, w2, nbad);
  else
    hipLaunchKernelGGL(k_repack_packed<16>, grid, blk, 0, nlg_stream(stream), wpk, out, cols, pk, fcount, wng, w2, nbad);
  NLG_LAUNCHED("repack base-4 codes to 2-bit");
  return NLG_OK;
}
