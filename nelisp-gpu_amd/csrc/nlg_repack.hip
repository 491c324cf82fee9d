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

#include <mutex>
#include <unordered_map>

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
__device__ __forceinline__ uint32_t packed_word(const float *row, uint32_t cols, uint32_t pk, uint32_t fcount,
                                                uint32_t wi, uint32_t &bad) {
  const uint32_t f0 = 16 * wi / pk;
  uint32_t pv[NF];
#pragma unroll
  for (int j = 0; j < NF; j++) {
    const uint32_t fi = f0 + j < fcount ? f0 + j : fcount - 1;
    pv[j] = nlg_f2u(row[fi]);
  }
  uint32_t word = 0, z = 16 * wi - f0 * pk, j = 0;
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
  return word;
}

template <int NF>
__global__ __launch_bounds__(256) void k_repack_packed(const float *wpk, uint32_t out, uint32_t cols, uint32_t pk,
                                                       uint32_t fcount, uint32_t wng, uint32_t *w2, uint32_t *nbad) {
  const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (uint64_t)out * wng) return;
  const uint32_t o = (uint32_t)(idx / wng), wi = (uint32_t)(idx % wng);
  uint32_t bad = 0;
  w2[idx] = packed_word<NF>(wpk + (size_t)o * fcount, cols, pk, fcount, wi, bad);
  if (nbad && bad) atomicAdd(nbad, bad);
}

// pk = 12 (codes below 4^12 = 2^24, exact in f32): four floats hold 48 codes,
// three 2-bit words.  Code c sits in bits 2z, 2z+1 (lo, hi) and the 2-bit
// field of c - 1 is (~lo, ~(lo | hi)) bit for bit -- 0 -> 11, 1 -> 00,
// 2 -> 01, and the unrepresentable 3 -> 00 like the per-word path -- so a
// float's twelve fields are five bitwise operations, and the three words
// are shifts of the four.  One thread per 48-column group of a row; a row's
// last, partial group takes the per-word path.
__device__ __forceinline__ uint32_t fields12(uint32_t u, uint32_t &bad) {
  const uint32_t lo = u & 0x555555u, hi = (u >> 1) & 0x555555u;
  bad += __builtin_popcount(lo & hi);
  return (~lo & 0x555555u) | ((~(lo | hi) & 0x555555u) << 1);
}

// W32: out * ngr < 2^32, so the index splits with a 32-bit division
template <bool W32>
__global__ __launch_bounds__(256) void k_repack_pk12(const float *wpk, uint32_t out, uint32_t cols, uint32_t fcount,
                                                     uint32_t wng, uint32_t ngr, uint32_t *w2, uint32_t *nbad) {
  uint32_t o, gi;
  if (W32) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= out * ngr) return;
    o = idx / ngr;
    gi = idx - o * ngr;
  } else {
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)out * ngr) return;
    o = (uint32_t)(idx / ngr);
    gi = (uint32_t)(idx % ngr);
  }
  const float *row = wpk + (size_t)o * fcount;
  uint32_t *dst = w2 + (size_t)o * wng + 3 * gi;
  uint32_t bad = 0;
  if (48 * gi + 48 <= cols && 4 * gi + 4 <= fcount) {
    // one 16-byte load and one 12-byte store (rows are only 4-byte aligned;
    // global memory takes unaligned vector accesses)
    float v[4];
    __builtin_memcpy(v, row + 4 * gi, sizeof v);
    const uint32_t f0 = fields12(nlg_f2u(v[0]), bad), f1 = fields12(nlg_f2u(v[1]), bad);
    const uint32_t f2 = fields12(nlg_f2u(v[2]), bad), f3 = fields12(nlg_f2u(v[3]), bad);
    const uint32_t wo[3] = {f0 | (f1 << 24),          // columns 0..15: float 0 codes 0..11, float 1 codes 0..3
                            (f1 >> 8) | (f2 << 16),   // columns 16..31: float 1 codes 4..11, float 2 codes 0..7
                            (f2 >> 16) | (f3 << 8)};  // columns 32..47: float 2 codes 8..11, float 3 codes 0..11
    __builtin_memcpy(dst, wo, sizeof wo);
  } else {
    for (uint32_t k = 0; k < 3 && 3 * gi + k < wng; k++) dst[k] = packed_word<5>(row, cols, 12, fcount, 3 * gi + k, bad);
  }
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
  nlg_tiled_refresh_range(w2, (size_t)out * ((cols + 15) / 16) * 4, nlg_stream(stream));
  NLG_LAUNCHED("tiled-copy refresh");
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
  if (pk == 12) {
    const uint32_t ngr = (wng + 2) / 3;
    const uint64_t ng = (uint64_t)out * ngr;
    const dim3 g12((unsigned)((ng + 255) / 256));
    if (ng + 255 < (1ull << 32))
      hipLaunchKernelGGL(k_repack_pk12<true>, g12, blk, 0, nlg_stream(stream), wpk, out, cols, fcount, wng, ngr, w2, nbad);
    else
      hipLaunchKernelGGL(k_repack_pk12<false>, g12, blk, 0, nlg_stream(stream), wpk, out, cols, fcount, wng, ngr, w2, nbad);
  } else if (pk >= 4)
    hipLaunchKernelGGL(k_repack_packed<5>, grid, blk, 0, nlg_stream(stream), wpk, out, cols, pk, fcount, wng, w2, nbad);
  else
    hipLaunchKernelGGL(k_repack_packed<16>, grid, blk, 0, nlg_stream(stream), wpk, out, cols, pk, fcount, wng, w2, nbad);
  NLG_LAUNCHED("repack base-4 codes to 2-bit");
  nlg_tiled_refresh_range(w2, (size_t)out * wng * 4, nlg_stream(stream));
  NLG_LAUNCHED("tiled-copy refresh");
  return NLG_OK;
}

// ------------------------------------------------------------ tiled copies
//
// The prefill GEMM (k_tgemm_w) hands lane 32g + i of a wave the words
// 8g..8g+7 of row i's 256-column chunk: 32 bytes of each of 32 rows, so a
// load instruction over the row layout touches 32 cache lines and uses a
// quarter of each.  The tiled copy stores each (32-row block, chunk) as one
// 2 KiB tile in exactly that order: 16-byte unit u = 64h + 32g + i of tile
// (b, c) is words 16c + 8g + 4h .. +3 of row 32b + i (zero past the last
// row), and the tiles of a row block follow each other chunk by chunk.  The
// wave's two loads of a chunk then read units lane and 64 + lane: 1 KiB
// each, contiguous.  Same bits as the row layout, reordered.

namespace {

__global__ __launch_bounds__(256) void k_tile_2bit(const uint32_t *w2, uint32_t rows, uint32_t wng, uint32_t nch,
                                                   uint64_t nunits, uint4 *wt) {
  const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= nunits) return;
  const uint32_t u = (uint32_t)idx & 127u;
  const uint64_t tile = idx >> 7;
  const uint32_t c = (uint32_t)(tile % nch), b = (uint32_t)(tile / nch);
  const uint32_t i = u & 31u, g = (u >> 5) & 1u, h = u >> 6;
  const uint32_t row = 32 * b + i;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row < rows) v = *(const uint4 *)(w2 + (size_t)row * wng + 16 * c + 8 * g + 4 * h);
  wt[idx] = v;
}

struct TiledCopy {
  uint32_t rows, cols;
  uint32_t *wt;
  size_t bytes() const { return (size_t)rows * (cols / 16) * 4; }  // the row layout it copies
};
std::mutex g_tiled_mu;
std::unordered_map<const uint32_t *, TiledCopy> g_tiled;
size_t g_tiled_n = 0;  // entries, read without the lock as a fast "none" test

}  // namespace

size_t nlg_tiled_bytes(uint32_t rows, uint32_t cols) { return (size_t)((rows + 31) / 32) * 32 * (cols / 4); }

const uint32_t *nlg_tiled_find(const uint32_t *w2, uint32_t rows, uint32_t cols) {
  if (!__atomic_load_n(&g_tiled_n, __ATOMIC_RELAXED)) return nullptr;
  std::lock_guard<std::mutex> lk(g_tiled_mu);
  const auto it = g_tiled.find(w2);
  return it != g_tiled.end() && it->second.rows == rows && it->second.cols == cols ? it->second.wt : nullptr;
}

// Writes into registered weights through the library (uploads, device
// copies, fills, repacks) refresh the copies they touch, in stream order
// after the write, in place (a captured graph keeps reading the same copy).
void nlg_tiled_refresh_range(const void *dst, size_t bytes, hipStream_t st) {
  if (!bytes || !__atomic_load_n(&g_tiled_n, __ATOMIC_RELAXED)) return;
  const uintptr_t lo = (uintptr_t)dst, hi = lo + bytes;
  std::lock_guard<std::mutex> lk(g_tiled_mu);
  for (auto &kv : g_tiled) {
    const uintptr_t a = (uintptr_t)kv.first, b = a + kv.second.bytes();
    if (a >= hi || b <= lo) continue;
    const uint32_t nch = kv.second.cols / 256;
    const uint64_t nunits = nlg_tiled_bytes(kv.second.rows, kv.second.cols) / 16;
    hipLaunchKernelGGL(k_tile_2bit, dim3((unsigned)((nunits + 255) / 256)), dim3(256), 0, st, kv.first,
                       kv.second.rows, kv.second.cols / 16, nch, nunits, (uint4 *)kv.second.wt);
  }
}

// Freeing device memory drops the copies of every registration inside it
// (a later allocation at the same address must not meet a stale copy).
void nlg_tiled_drop_range(const void *base, size_t bytes) {
  if (!__atomic_load_n(&g_tiled_n, __ATOMIC_RELAXED)) return;
  const uintptr_t lo = (uintptr_t)base, hi = lo + (bytes ? bytes : 1);
  std::lock_guard<std::mutex> lk(g_tiled_mu);
  for (auto it = g_tiled.begin(); it != g_tiled.end();) {
    const uintptr_t a = (uintptr_t)it->first;
    if (a >= lo && a < hi) {
      (void)hipFree(it->second.wt);
      it = g_tiled.erase(it);
    } else {
      ++it;
    }
  }
  __atomic_store_n(&g_tiled_n, g_tiled.size(), __ATOMIC_RELAXED);
}

void nlg_tiled_release_all(void) {
  std::lock_guard<std::mutex> lk(g_tiled_mu);
  for (auto &kv : g_tiled) (void)hipFree(kv.second.wt);
  g_tiled.clear();
  __atomic_store_n(&g_tiled_n, 0, __ATOMIC_RELAXED);
}

extern "C" int nlg_ternary_tiled_register(const uint32_t *w2, uint32_t rows, uint32_t cols, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!w2) return nlg_fail("tiled weights: null weights");
  if (!rows || !cols || cols % 256) return nlg_fail("tiled weights: rows must be nonzero, cols a multiple of 256");
  if ((uintptr_t)w2 & 15) return nlg_fail("tiled weights: w2 must be 16-byte aligned");
  const size_t bytes = nlg_tiled_bytes(rows, cols);
  uint32_t *wt = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_tiled_mu);
    auto it = g_tiled.find(w2);
    if (it != g_tiled.end() && it->second.rows == rows && it->second.cols == cols) wt = it->second.wt;
  }
  const bool fresh = !wt;
  if (fresh) {
    const hipError_t e = hipMalloc((void **)&wt, bytes);
    if (e != hipSuccess) return nlg_fail("tiled weights: hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
  }
  const uint32_t nch = cols / 256;
  const uint64_t nunits = bytes / 16;
  hipStream_t st = nlg_stream(stream);
  hipLaunchKernelGGL(k_tile_2bit, dim3((unsigned)((nunits + 255) / 256)), dim3(256), 0, st, w2, rows, cols / 16,
                     nch, nunits, (uint4 *)wt);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    if (fresh) (void)hipFree(wt);
    return nlg_fail("tiled weights: %s", hipGetErrorString(e));
  }
  if (fresh) {
    std::lock_guard<std::mutex> lk(g_tiled_mu);
    auto it = g_tiled.find(w2);
    if (it != g_tiled.end()) (void)hipFree(it->second.wt);  // another shape before
    g_tiled[w2] = TiledCopy{rows, cols, wt};
    __atomic_store_n(&g_tiled_n, g_tiled.size(), __ATOMIC_RELAXED);
  }
  return NLG_OK;
}

extern "C" int nlg_ternary_tiled_unregister(const uint32_t *w2) {
  std::lock_guard<std::mutex> lk(g_tiled_mu);
  auto it = g_tiled.find(w2);
  if (it == g_tiled.end()) return NLG_OK;
  const hipError_t e = hipFree(it->second.wt);
  g_tiled.erase(it);
  __atomic_store_n(&g_tiled_n, g_tiled.size(), __ATOMIC_RELAXED);
  if (e != hipSuccess) return nlg_fail("tiled weights: hipFree failed: %s", hipGetErrorString(e));
  return NLG_OK;
}
