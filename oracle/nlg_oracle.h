/* nlg_oracle.h -- CPU restatement of nelisp-gpu's hot-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X kernels and the CPU baseline timed by bench.py; it is never linked
 * into, loaded by, or called from the product library (libnlgpu) or the CLI
 * hosts.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Each kernel is restated from its DSL body in lisp/nelisp-gpu-kernels.el
 * (line cited per function in nlg_oracle.c), following the op semantics of
 * lisp/nelisp-gpu-compile.el: uint arithmetic wraps mod 2^32, integer
 * compares are unsigned, float ops are single IEEE operations evaluated in
 * the body's order with no contraction (built with -ffp-contract=off),
 * `(uint f)` truncates toward zero, and every float reduction is serial in
 * index order.  Buffer access is robust: a read past a buffer's end gives 0
 * and a write past it is dropped (Vulkan robustBufferAccess), so a malformed
 * request can never crash the checker.
 */
#ifndef NLG_ORACLE_H
#define NLG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Run kernel `name` over `groups` workgroups of 64 invocations (256 for
 * matmul-tiled), exactly as its DSL body would.  bufs[i] has sizes[i]
 * 4-byte elements.  Returns 0, or 1 for an unknown name or a wrong number of
 * buffers/push constants. */
int or_dispatch(const char *name, float **bufs, const uint32_t *sizes, uint32_t nbuf,
                const uint32_t *push, uint32_t npush, uint32_t groups);
int or_kernel_count(void);
const char *or_kernel_name(int i);
int or_kernel_abi(const char *name, uint32_t *nbuf, uint32_t *npush);

/* The composite ternary x int8 linear (see nlgpu.h nlg_ternary_linear_i8):
 * 2-bit fields unpacked to int8 lanes, then bitlinear-dp4a-1f's int32 sdot
 * accumulation and fp32 epilogue.  bias may be NULL. */
void or_ternary_linear_i8(const uint32_t *xq, const float *gamma, const uint32_t *w2,
                          const float *bias, const float *beta, int beta_per_row, float *y,
                          uint32_t seq, uint32_t out, uint32_t cols);
/* Same, returning the exact int32 accumulators instead of y. */
void or_ternary_acc_i8(const uint32_t *xq, const uint32_t *w2, int32_t *acc, uint32_t seq,
                       uint32_t out, uint32_t cols);
/* pack-act-rows over `seq` rows of `cols` (kernels.el:884-932). */
void or_pack_act_rows(const float *x, uint32_t *xq, float *gamma, uint32_t seq, uint32_t cols);
/* softmax over rows (kernels.el:28-42); c may equal a. */
void or_softmax_rows(const float *a, float *c, uint32_t rows, uint32_t cols);

/* rmsnorm-istd + rmsnorm-fwd (kernels.el:1249-1265) with eps a parameter. */
void or_rmsnorm_rows(const float *x, const float *gain, float eps, float *y, uint32_t rows,
                     uint32_t cols);
/* decode-attn-b (kernels.el:366-390) over fp16 caches [B][kvheads][max_seq][hd]. */
void or_decode_attn_f16(const float *q, const uint16_t *kc, const uint16_t *vc, uint32_t pos,
                        float *out, uint32_t B, uint32_t heads, uint32_t kvheads, uint32_t hd,
                        uint32_t max_seq);

/* decode-attn-paged-v (kernels.el:1222-1246) over fp16 pools
 * [block][bs][kvheads][hd]; sequence s at position lens[s] (negative: 0);
 * table [B x mbps]; blocks outside [0, npool) read as zero rows. */
void or_decode_attn_paged_f16(const float *q, const uint16_t *kp, const uint16_t *vp, const int32_t *lens,
                              const int32_t *table, uint32_t npool, float *out, uint32_t B, uint32_t heads,
                              uint32_t kvheads, uint32_t hd, uint32_t bs, uint32_t mbps);

/* decode-attn-stream (kernels.el:404-451) over fp16 ring caches
 * [B][kvheads][nsink + win][hd]; sequence s at stream position pos[s]
 * (negative: 0); co/si: [>= nsink + win][hd/2] rotation tables. */
void or_decode_attn_stream_f16(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *pos,
                               const float *co, const float *si, float *out, uint32_t B, uint32_t heads,
                               uint32_t kvheads, uint32_t hd, uint32_t nsink, uint32_t win);
/* attn-stream-entries (kernels.el:1052-1090) over fp16 caches
 * [B][kvheads][nslots][hd]; ent [B][ne][2] int32 (slot, rank); qrank [B];
 * co/si [trows][hd/2]; bad slots read zero rows, bad ranks zero rotations. */
void or_attn_entries_f16(const float *q, const uint16_t *kc, const uint16_t *vc, const int32_t *ent,
                         const int32_t *qrank, const float *co, const float *si, float *out, uint32_t B,
                         uint32_t heads, uint32_t kvheads, uint32_t hd, uint32_t nslots, uint32_t ne,
                         uint32_t trows);

/* Weight ingest into the 2-bit layout of ternary-rows (kernels.el:700-746:
 * field f of word w = column 16w+f, bits 2f..2f+1, sign-extended).
 * From int8 lanes (bitlinear-dp4a-1f/-rows WP, kernels.el:619-653: lane l of
 * word g = column 4g+l, signed byte): lanes outside [-2, 1] become 0 and are
 * counted.  From base-4 codes in f32 values (bitlinear-packed(-v),
 * kernels.el:992-1040: packed = (uint WPK[o*fcount+f]), column f*pk+z has
 * code (packed/4^z)%4, weight code-1; no weight past fcount*pk): code 3
 * becomes 0 and is counted.  Return: the count. */
uint32_t or_repack_i8_2bit(const uint32_t *wp, uint32_t out, uint32_t cols, uint32_t *w2);
uint32_t or_repack_packed_2bit(const float *wpk, uint32_t out, uint32_t cols, uint32_t pk, uint32_t fcount,
                               uint32_t *w2);

/* Number of OpenMP threads the parallel loops use (1 when built without
 * OpenMP); set_threads(0) keeps the runtime default. */
int or_threads(void);
void or_set_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
