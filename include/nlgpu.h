/* nlgpu.h -- C ABI of the MI355X (gfx950) implementation of nelisp-gpu's
 * quantized-LLM kernel path.
 *
 * Everything here is plain C: device pointers are `void*` / typed pointers,
 * sizes are integers, streams are opaque `void*` (a hipStream_t; NULL means
 * the library's own stream).  No HIP or torch type appears in a signature, so
 * the CLI hosts (vkserver, vkrun, vkmatmul, vksoftmax, vkcompute) and any
 * FFI (ctypes, cgo, an Emacs module) can bind it directly.
 *
 * Every function returns NLG_OK (0) on success and NLG_ERR (1) on failure,
 * with a message available from nlg_last_error().  No function exits the
 * process; the CLI hosts decide what a failure means for them.
 *
 * Reference interfaces replaced (paths under zawatton/nelisp-gpu):
 *   device bring-up        host/vkserver.c:213-245 (init_vulkan),
 *                          host/vkcompute.c:90-100 (NELISP_GPU_DEVICE policy)
 *   buffers                host/vkserver.c:126-149 (make_buffer_ex),
 *                          :169-205 (staged_write), :207-211 (write_buffer)
 *   kernel by name         host/vkserver.c:247-272 (get_kernel),
 *                          :312-322 (record + submit one dispatch)
 *   fused batch / compiled host/vkserver.c:437-506 (handle_batch),
 *                          :511-604 (handle_compile / handle_run_compiled)
 *   kernel semantics       lisp/nelisp-gpu-kernels.el (one entry per name)
 */
#ifndef NLGPU_H
#define NLGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NLG_OK 0
#define NLG_ERR 1

/* ------------------------------------------------------------------------
 * Device, memory, streams
 * ---------------------------------------------------------------------- */

/* Select and initialise the GPU.  device < 0 applies the reference policy:
 * env NELISP_GPU_DEVICE if set, else device 0 (every MI355X is discrete).
 * Replaces host/vkserver.c:213-245 and host/vkcompute.c:90-100.  Idempotent. */
int nlg_init(int device);
/* Release the library's stream, staging and graph objects. */
int nlg_shutdown(void);
/* Message for the most recent failure on this thread ("" if none). */
const char *nlg_last_error(void);
/* Marketing name of the active device (e.g. "AMD Instinct MI355X"). */
int nlg_device_name(char *buf, size_t len);
/* Number of compute units and the active device's gfx name. */
int nlg_device_info(int *num_cu, char *arch, size_t arch_len);

/* Device memory, zero-filled.  Replaces make_buffer_ex (vkserver.c:126-149):
 * every buffer lives in HBM (no HOST_VISIBLE fallback is needed with 288 GB).
 * Returns NULL on failure. */
void *nlg_malloc(size_t bytes);
int nlg_free(void *dev);
/* Synchronous copies (host memory may be pageable).  Replaces write_buffer /
 * staged_write (vkserver.c:169-211) and the map-and-fwrite read-back
 * (vkserver.c:325-330). */
int nlg_upload(void *dev_dst, const void *host_src, size_t bytes);
int nlg_download(void *host_dst, const void *dev_src, size_t bytes);
int nlg_copy_d2d(void *dev_dst, const void *dev_src, size_t bytes, void *stream);
/* Zero `bytes` of device memory with a fill kernel (safe inside a captured
 * graph, unlike a runtime memset).  Replaces vkCmdFillBuffer (vkserver.c:554-556). */
int nlg_zero(void *dev, size_t bytes, void *stream);
/* Read `bytes` at `offset` of `path` into device memory through pinned
 * staging.  *missing receives the number of bytes the file could not supply
 * (the tail of dev is then zero).  Replaces handle_upload_file's
 * fread+staged_write (vkserver.c:371-410). */
int nlg_upload_file(void *dev_dst, const char *path, uint64_t offset, size_t bytes,
                    size_t *missing);

void *nlg_stream_create(void);
/* Waits for the stream, releases the scratch the batched linears keep per
 * stream, and destroys it (a graph captured on it must not run afterwards). */
int nlg_stream_destroy(void *stream);
int nlg_stream_sync(void *stream);
/* The library's default stream (what NULL means). */
void *nlg_default_stream(void);

/* Device-side timing: events recorded on a stream. */
void *nlg_event_create(void);
int nlg_event_destroy(void *ev);
int nlg_event_record(void *ev, void *stream);
int nlg_event_elapsed_ms(void *start, void *stop, float *ms);

/* ------------------------------------------------------------------------
 * Kernels by name: the lisp/nelisp-gpu-kernels.el ABI
 * ---------------------------------------------------------------------- */

/* One buffer binding: a device pointer and its length in 4-byte elements
 * (the reference's "float count"; packed words ride in the same slots). */
typedef struct {
  void *ptr;
  uint32_t nfloats;
} nlg_buffer;

/* Number of kernel names the library implements, their names, and the
 * binding/push-constant counts each expects (Appendix-A order of
 * lisp/nelisp-gpu-kernels.el :buffers and :push). */
int nlg_kernel_count(void);
const char *nlg_kernel_name(int index);
int nlg_kernel_lookup(const char *name);
int nlg_kernel_abi(const char *name, uint32_t *nbuf, uint32_t *npush);

/* Run kernel `name` as the reference would run `groups` workgroups of 64
 * invocations: every invocation gid < min(domain, 64*groups) does the work
 * its DSL body defines.  Buffers are checked against the extents the push
 * constants imply before anything is launched (status NLG_ERR, nothing run, if
 * a buffer is short); data-dependent indices (POS, TOK, TABLE) are bounds-
 * checked on the device (out-of-range reads give 0, writes are dropped).
 * Replaces get_kernel (vkserver.c:247-272) plus one vkCmdDispatch
 * (vkserver.c:312-322, vkrun.c:117-123). */
int nlg_dispatch(const char *name, const nlg_buffer *bufs, uint32_t nbuf,
                 const uint32_t *push, uint32_t npush, uint32_t groups, void *stream);

/* ------------------------------------------------------------------------
 * Graphs: a recorded sequence of launches replayed with one call.
 * Replaces OP_COMPILE / OP_RUN_COMPILED / OP_FREE_COMPILED
 * (vkserver.c:511-615).  Capture is stream capture: everything launched on
 * `stream` between begin and end is recorded, not executed.
 * ---------------------------------------------------------------------- */
int nlg_graph_begin(void *stream);
int nlg_graph_end(void *stream, void **graph_exec);
int nlg_graph_launch(void *graph_exec, void *stream);
int nlg_graph_destroy(void *graph_exec);

/* ------------------------------------------------------------------------
 * Typed hot path (device pointers)
 * ---------------------------------------------------------------------- */

/* Per-row absmax int8 quantisation + packing.  gamma[r] = max|x[r,:]| / 127;
 * lane = uint(|x/gamma| + 0.5) clamped to 127, negatives stored as 256-lane;
 * four lanes per u32 word, lane l in bits 8l..8l+7; ng = ceil(cols/4) words
 * per row.  Bit-identical to `pack-act-rows` (lisp/nelisp-gpu-kernels.el:884-932). */
int nlg_pack_act_rows(const float *x, uint32_t *xq, float *gamma, uint32_t seq,
                      uint32_t cols, void *stream);

/* Ternary 2-bit weights x int8 activations, int32 accumulation, fp32 epilogue:
 *   acc[s,o] = sum_c decode(W[o,c]) * int8(xq[s,c])         (exact int32)
 *   y[s,o]   = bias[o] + (beta[b] * gamma[s]) * (float)acc  (IEEE, no FMA)
 * with b = o when beta_per_row, else 0.  W is the reference's 2-bit format:
 * row-major, wng = ceil(cols/16) u32 words per row, field f of a word in bits
 * 2f..2f+1, 00->0 01->+1 11->-1 10->-2 (ternary-rows, kernels.el:700-746).
 * The accumulation and epilogue are bitlinear-dp4a-1f's (kernels.el:619-634)
 * on the 2-bit weights unpacked to int8 lanes.  bias may be NULL (zero).
 * Requires cols <= 131072 (int32 headroom of the x64-scaled partial sums). */
int nlg_ternary_linear_i8(const uint32_t *xq, const float *gamma, const uint32_t *w2,
                          const float *bias, const float *beta, int beta_per_row,
                          float *y, uint32_t seq, uint32_t out, uint32_t cols,
                          void *stream);

/* Launch-geometry variant of nlg_ternary_linear_i8 for tuning sweeps:
 * rows_per_wave in {1,2,4,8}, waves_per_block in 1..4.  Results are
 * bit-identical for every geometry. */
int nlg_ternary_linear_i8_cfg(const uint32_t *xq, const float *gamma, const uint32_t *w2,
                              const float *bias, const float *beta, int beta_per_row, float *y,
                              uint32_t seq, uint32_t out, uint32_t cols, int rows_per_wave,
                              int waves_per_block, void *stream);

/* The whole ternary linear from f32 activations: pack-act-rows quantisation
 * of x then nlg_ternary_linear_i8, bit-identical to running the two.  When
 * cols % 64 == 0, cols <= 16384 and seq <= 3 (seq <= 4 when cols % 256 != 0)
 * it is one launch (each workgroup quantises the row into LDS while its
 * weight loads are in flight) and needs no workspace; with 4 or more tokens
 * and cols % 256 == 0 it takes the batched form below (library scratch, no
 * workspace); otherwise it runs pack-act-rows into `workspace`
 * (nlg_ternary_linear_workspace bytes) and then the GEMV.
 * gamma_out (may be NULL) receives the per-token scales. */
int nlg_ternary_linear(const float *x, const uint32_t *w2, const float *bias, const float *beta,
                       int beta_per_row, float *y, float *gamma_out, uint32_t seq, uint32_t out,
                       uint32_t cols, void *workspace, size_t workspace_bytes, void *stream);
size_t nlg_ternary_linear_workspace(uint32_t seq, uint32_t cols);

/* nlg_ternary_linear for callers that cannot allocate (code under graph
 * capture, tight serving loops): same results, bit for bit, with no
 * workspace argument and no device allocation on any path.  Whatever
 * scratch the form needs (packed activations for the two-launch form, int8
 * activations and scales for the batched form) is a fixed array of
 * NLG_NOALLOC_SCRATCH_BYTES that the library holds on each GPU until the
 * process ends; shapes needing more (about seq x cols > 16.7 M) fail with
 * NLG_ERR and launch nothing.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, concurrent graph
 * replays) race and must not be issued.  No reference counterpart. */
#define NLG_NOALLOC_SCRATCH_BYTES (16u << 20)
int nlg_ternary_linear_noalloc(const float *x, const uint32_t *w2, const float *bias, const float *beta,
                               int beta_per_row, float *y, float *gamma_out, uint32_t seq, uint32_t out,
                               uint32_t cols, void *stream);
/* Tuning variant: rows_per_wave in {1,2,4} for the one-launch form (0 = default). */
int nlg_ternary_linear_cfg(const float *x, const uint32_t *w2, const float *bias, const float *beta,
                           int beta_per_row, float *y, float *gamma_out, uint32_t seq, uint32_t out,
                           uint32_t cols, int rows_per_wave, void *workspace, size_t workspace_bytes,
                           void *stream);

/* Row softmax, numerically stable (row max subtracted), in place when
 * c == a.  Semantics of `softmax` (kernels.el:28-42). */
int nlg_softmax_rows(const float *a, float *c, uint32_t rows, uint32_t cols, void *stream);

/* ------------------------------------------------------------------------
 * Decoder-layer fusions.  The reference runs a decode layer as a chain of
 * named kernels over resident buffers (rmsnorm-istd, rmsnorm-fwd,
 * pack-act-rows, the linear, decode-rope, cache-append, decode-attn,
 * silu-mul, add2); each entry point below is one launch doing a run of that
 * chain, with the same per-element arithmetic.  All require
 * cols % 64 == 0, cols <= 16384 and 16-byte aligned x, gain and weights.
 * The RMSNorm is rmsnorm-istd + rmsnorm-fwd (kernels.el:1249-1265) with eps
 * a parameter: S = 1/sqrt(sum(x*x)/cols + eps), xn = (x*S)*gain; its sum is
 * a tree, so S may differ from the serial loop's in the last bit.
 * With 4 or more tokens and cols % 256 == 0 each of them (and
 * nlg_ternary_linear) runs as per-token quantisation into library scratch
 * followed by the int8 matrix-core GEMM.  That scratch is one per stream:
 * calls on different streams may overlap.  It grows by allocating, so on a
 * stream being captured into a graph it must already be large enough (make
 * the call once on that stream first).  A captured graph keeps using the
 * scratch of the stream it was captured on: do not replay it while other
 * batched calls on that stream, or another replay of it, may run.
 * ---------------------------------------------------------------------- */

/* y = linear(rmsnorm(x)) (rmsnorm-istd, rmsnorm-fwd, pack-act-rows,
 * bitlinear-dp4a-1f on 2-bit weights). */
int nlg_rms_ternary_linear(const float *x, const float *gain, float eps, const uint32_t *w2,
                           const float *bias, const float *beta, int beta_per_row, float *y,
                           uint32_t seq, uint32_t out, uint32_t cols, void *stream);

/* y = res + linear(x) (pack-act-rows, the linear, add2 kernels.el:812-821);
 * res may equal y (the residual stream updated in place). */
int nlg_ternary_linear_residual(const float *x, const uint32_t *w2, const float *bias,
                                const float *beta, int beta_per_row, const float *res, float *y,
                                uint32_t seq, uint32_t out, uint32_t cols, void *stream);

/* SwiGLU: w2gu holds 2*dff rows, row 2j = gate row j, row 2j+1 = up row j;
 * g, u = linear(rmsnorm(x)); h[j] = (g * (1/(1 + exp(0 - g)))) * u
 * (silu-mul, kernels.el:186-193).  beta indexes the interleaved rows.
 * gain NULL: no RMSNorm (g, u = linear(x)). */
int nlg_rms_ternary_swiglu(const float *x, const float *gain, float eps, const uint32_t *w2gu,
                           const float *beta, int beta_per_row, float *h, uint32_t seq,
                           uint32_t dff, uint32_t cols, void *stream);

/* Attention input projection at decode: rows of w2qkv are q (heads*head_dim)
 * | k (kvheads*head_dim) | v.  q and k are rotated at position pos[0]
 * (decode-rope / decode-rope-b, kernels.el:291-306, :340-355: pairs (2m,
 * 2m+1) of each head, C0 = a0*cos - a1*sin, C1 = a0*sin + a1*cos with
 * tables [max_seq x head_dim/2]); q goes to `q` [seq x heads*head_dim]; k
 * and v are rounded to fp16 and stored at position pos[0] of the caches
 * (cache-append-b, kernels.el:356-365), laid out [seq][kvheads][max_seq]
 * [head_dim].  A pos[0] outside [0, max_seq) stores nothing to the caches. */
int nlg_rms_ternary_qkv_rope(const float *x, const float *gain, float eps, const uint32_t *w2qkv,
                             const float *beta, int beta_per_row, float *q, uint16_t *kcache,
                             uint16_t *vcache, const float *rope_cos, const float *rope_sin,
                             const int32_t *pos, uint32_t seq, uint32_t heads, uint32_t kvheads,
                             uint32_t head_dim, uint32_t max_seq, uint32_t cols, void *stream);
/* The same for a whole prompt (the prefill rows nlg_prefill_attn_f16 reads):
 * row r of x is sequence r / qper at position pos[0] + r % qper; q of row r
 * is rotated at that position and k, v go to that position of sequence
 * r / qper's caches [rows/qper][kvheads][max_seq][head_dim].  Rows whose
 * position lies outside [0, max_seq) store nothing to the caches.  rows must
 * be a multiple of qper > 0.  The reference runs a prompt as decode-rope-b /
 * cache-append-b per position (kernels.el:340-365); this is those steps for
 * every position at once. */
int nlg_rms_ternary_qkv_rope_prompt(const float *x, const float *gain, float eps, const uint32_t *w2qkv,
                                    const float *beta, int beta_per_row, float *q, uint16_t *kcache,
                                    uint16_t *vcache, const float *rope_cos, const float *rope_sin,
                                    const int32_t *pos, uint32_t rows, uint32_t qper, uint32_t heads,
                                    uint32_t kvheads, uint32_t head_dim, uint32_t max_seq, uint32_t cols,
                                    void *stream);

/* LM head + greedy choice: logits = linear(rmsnorm(x)) and argmax[s] = the
 * lowest index of the largest logit (NaN never chosen; -1 if none). */
int nlg_rms_ternary_argmax(const float *x, const float *gain, float eps, const uint32_t *w2,
                           const float *beta, int beta_per_row, float *logits, int32_t *argmax,
                           uint32_t seq, uint32_t vocab, uint32_t cols, void *workspace,
                           size_t workspace_bytes, void *stream);
size_t nlg_rms_ternary_argmax_workspace(uint32_t seq, uint32_t vocab);

/* Single-query GQA attention over fp16 caches [batch][kvheads][max_seq]
 * [head_dim] for positions 0..pos[0]: decode-attn-b's arithmetic
 * (kernels.el:366-390: s = (q.k)/sqrt(head_dim), e = exp(s - max),
 * out = sum(e*v)/sum(e)) with K, V read as fp16.  head_dim 64 or 128,
 * heads/kvheads in {1,2,4,8}.  Two launches: chunks of positions scored
 * in parallel into `workspace` (nlg_decode_attn_f16_workspace bytes), then
 * merged. */
int nlg_decode_attn_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                        const int32_t *pos, float *out, uint32_t batch, uint32_t heads,
                        uint32_t kvheads, uint32_t head_dim, uint32_t max_seq, void *workspace,
                        size_t workspace_bytes, void *stream);
size_t nlg_decode_attn_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                     uint32_t head_dim, uint32_t max_seq);

/* Paged fp16 KV (PagedAttention): decode-attn-paged-v's arithmetic
 * (kernels.el:1222-1246) over pools [block][bs][kvheads][head_dim] fp16
 * shared by all sequences; sequence b attends positions 0..lens[b] through
 * its row of the block table [batch x mbps] (position p in block
 * table[b*mbps + p/bs], offset p%bs), so sequences of different lengths and
 * shared prefix blocks mix in one batch.  Table entries outside
 * [0, npool) read as zero K/V rows.  Same chunk pass and merge as
 * nlg_decode_attn_f16; workspace from nlg_decode_attn_paged_f16_workspace. */
int nlg_decode_attn_paged_f16(const float *q, const uint16_t *kpool, const uint16_t *vpool,
                              const int32_t *lens, const int32_t *table, uint32_t npool, float *out,
                              uint32_t batch, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                              uint32_t bs, uint32_t mbps, void *workspace, size_t workspace_bytes,
                              void *stream);
size_t nlg_decode_attn_paged_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                           uint32_t head_dim, uint32_t bs, uint32_t mbps);
/* cache-append-paged-v (kernels.el:1211-1220) into an fp16 pool: row b of
 * src [batch x kvdim] f32 goes to position lens[b] of sequence b (round to
 * nearest even); positions or blocks out of range are skipped. */
int nlg_cache_append_paged_f16(const float *src, const int32_t *lens, const int32_t *table, uint32_t npool,
                               uint16_t *pool, uint32_t batch, uint32_t kvdim, uint32_t bs, uint32_t mbps,
                               void *stream);

/* StreamingLLM fp16 ring caches: decode-attn-stream's arithmetic
 * (kernels.el:404-451) over caches [batch][kvheads][nsink + win][head_dim]
 * fp16 holding RAW (un-rotated) keys: nsink permanent sink slots, then a
 * win-slot ring.  Sequence b at stream position pos[b] (negative: 0) attends
 * len = min(pos + 1, nsink + win) cache-relative ranks: ranks below nsink
 * are the sink slots, later ones walk the ring from its oldest slot.  K of
 * rank r is rotated by rows r of co/si and q by row min(pos, nsink + win - 1)
 * (pairs (2m, 2m+1)); co/si hold >= nsink + win rows of head_dim/2 floats.
 * q, caches and tables 16-byte aligned; win > 0.  Same chunk pass and merge
 * as nlg_decode_attn_f16; workspace from nlg_decode_attn_stream_f16_workspace
 * (0 for invalid sizes). */
int nlg_decode_attn_stream_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                               const int32_t *pos, const float *co, const float *si, float *out,
                               uint32_t batch, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                               uint32_t nsink, uint32_t win, void *workspace, size_t workspace_bytes,
                               void *stream);
size_t nlg_decode_attn_stream_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads,
                                           uint32_t head_dim, uint32_t nsink, uint32_t win);
/* cache-append-ring (kernels.el:396-403) into fp16 ring caches: row b of src
 * [batch x kvheads*head_dim] f32 (raw K or V) goes to the slot of stream
 * position pos[b] (pos < nsink: slot pos; else nsink + (pos - nsink) mod
 * win), rounded to nearest even; negative positions write nothing. */
int nlg_cache_append_ring_f16(const float *src, const int32_t *pos, uint16_t *cache, uint32_t batch,
                              uint32_t kvheads, uint32_t head_dim, uint32_t nsink, uint32_t win,
                              void *stream);
/* attn-stream-entries (kernels.el:1052-1090) over fp16 caches
 * [batch][kvheads][nslots][head_dim]: sequence b attends the ne rows its
 * entry list names, ent[b] = ne (slot, cache-relative rank) int32 pairs
 * ([batch][ne][2], 8-byte aligned), K rotated by its rank and q by qrank[b]
 * through co/si ([trows][head_dim/2]).  Slots outside [0, nslots) read as
 * zero rows and ranks outside [0, trows) as zero rotations (the reference's
 * robust reads).  Workspace from nlg_attn_entries_f16_workspace. */
int nlg_attn_entries_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache, const int32_t *ent,
                         const int32_t *qrank, const float *co, const float *si, float *out, uint32_t batch,
                         uint32_t heads, uint32_t kvheads, uint32_t head_dim, uint32_t nslots, uint32_t ne,
                         uint32_t trows, void *workspace, size_t workspace_bytes, void *stream);
size_t nlg_attn_entries_f16_workspace(uint32_t batch, uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                                      uint32_t ne);
/* block-copy (kernels.el:1184-1193) on a K pool and a V pool of fp16 blocks
 * [npool][bs][kvdim] at once (copy-on-write of shared prefix blocks): n
 * copies in one launch, pairs[2i] -> pairs[2i+1]; pairs naming a block
 * outside [0, npool) are skipped.  Copies of one call run concurrently: no
 * destination may be another pair's source. */
int nlg_block_copy_f16(uint16_t *kpool, uint16_t *vpool, const int32_t *pairs, uint32_t n, uint32_t npool,
                       uint32_t bs, uint32_t kvdim, void *stream);

/* The first of nlg_decode_attn_f16's two launches alone: per chunk of
 * positions and head, the chunk's maximum score m (in base 2: q.k/sqrt(hd)
 * times log2 e), its sum of 2^(s - m) and the matching weighted sum of V,
 * left in `workspace` for nlg_attn_ternary_linear_residual. */
int nlg_decode_attn_f16_chunks(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                               const int32_t *pos, uint32_t batch, uint32_t heads, uint32_t kvheads,
                               uint32_t head_dim, uint32_t max_seq, void *workspace,
                               size_t workspace_bytes, void *stream);

/* The attention output projection with the chunk merge folded into it:
 * y = res + linear(attention), where attention is what nlg_decode_attn_f16
 * would return from the partials in `workspace` (bit-identical to running
 * that merge and then nlg_ternary_linear_residual).  One launch; needs
 * max_seq short enough for at most 4 chunks: max_seq <= 1024 at head_dim
 * 128, <= 2048 at 64 (longer caches: NLG_ERR, use the two calls above). */
int nlg_attn_ternary_linear_residual(const void *workspace, size_t workspace_bytes, uint32_t batch,
                                     uint32_t heads, uint32_t kvheads, uint32_t head_dim,
                                     uint32_t max_seq, const uint32_t *w2, const float *bias,
                                     const float *beta, int beta_per_row, const float *res, float *y,
                                     uint32_t out, void *stream);

/* Causal GQA attention for a whole prompt: attn-causal-gqa's arithmetic
 * (kernels.el:934-990: s = (q.k)/sqrt(head_dim) over positions 0..p,
 * ctx = sum(exp(s - max) v) / sum(exp(s - max))) over the fp16 caches
 * [rows/qper][kvheads][max_seq][head_dim] that nlg_rms_ternary_qkv_rope
 * fills.  q and ctx are [rows][heads*head_dim] f32; row r is sequence
 * r / qper at position pos[0] + r % qper.  head_dim 64 or 128, heads/kvheads
 * in {1,2,4,8}, rows a multiple of qper, one sequence's cache of one kv
 * head (max_seq x head_dim halves) under 2 GiB; f16 matrix cores with q and the
 * probabilities split into hi + lo halves (f32-grade products).  One launch,
 * or -- when the grid would have fewer than 256 workgroups (a single prompt)
 * -- two: the keys of each query block in pieces, then their merge, with the
 * pieces' partials in a scratch of the library kept per stream (grown on the
 * first such call; a call being captured that would have to grow it runs as
 * one launch instead).  Calls on one stream share that scratch, in stream
 * order. */
int nlg_prefill_attn_f16(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                         const int32_t *pos, uint32_t rows, uint32_t qper, uint32_t heads,
                         uint32_t kvheads, uint32_t head_dim, uint32_t max_seq, float *ctx,
                         void *stream);
/* That attention and the attention output projection with its residual:
 * y = res + linear(ctx) over rows x heads*head_dim (out rows of w2), the
 * prompt's counterpart of nlg_attn_ternary_linear_residual.  When the keys
 * are split (few prompts), the pieces are merged and quantised for the
 * projection in one launch; otherwise ctx_ws ([rows][heads*head_dim] f32)
 * receives the context on the way.  Bit-identical to nlg_prefill_attn_f16
 * followed by nlg_ternary_linear_residual.  The reference runs a prompt as
 * attn-causal-gqa, pack-act-rows, bitlinear-dp4a-1f and add2
 * (kernels.el:934-990, :884-932, :619-634, :812-821). */
int nlg_prefill_attn_ternary_linear_residual(const float *q, const uint16_t *kcache,
                                             const uint16_t *vcache, const int32_t *pos, uint32_t rows,
                                             uint32_t qper, uint32_t heads, uint32_t kvheads,
                                             uint32_t head_dim, uint32_t max_seq, float *ctx_ws,
                                             const uint32_t *w2, const float *bias, const float *beta,
                                             int beta_per_row, const float *res, float *y, uint32_t out,
                                             void *stream);

/* Weight ingest: the reference's other ternary formats repacked into the
 * 2-bit layout of ternary-rows (kernels.el:700-746) that every ternary entry
 * point here reads ([out x ceil(cols/16)] u32, 4x fewer bytes than int8
 * lanes, same int32 accumulators).  From int8 lanes: WP [out x ceil(cols/4)]
 * of bitlinear-dp4a-1f / -rows (kernels.el:619-653).  From base-4 codes:
 * WPK [out x fcount] f32 of bitlinear-packed / -v (kernels.el:992-1040),
 * pk codes per value (1..16).  A weight the 2-bit code cannot hold (an int8
 * lane outside [-2, 1], a base-4 code 3) is written as 0 and added to the
 * device counter *nbad (may be NULL).  One launch each, no host sync. */
int nlg_repack_i8_to_2bit(const uint32_t *wp, uint32_t out, uint32_t cols, uint32_t *w2, uint32_t *nbad,
                          void *stream);
int nlg_repack_packed_to_2bit(const float *wpk, uint32_t out, uint32_t cols, uint32_t pk, uint32_t fcount,
                              uint32_t *w2, uint32_t *nbad, void *stream);

/* Measurement (no counterpart in the reference, which times a submitted
 * command buffer from the host, vkmatmul.c:146-169): the bare one-token
 * linear of nlg_ternary_linear (no bias, one beta, no gamma output) whose
 * waves also write their start and end on the device's 100 MHz wall clock
 * to stamps ([waves][2] u64; nlg_ternary_linear_timed_stamps(out) bytes):
 * the kernel's device-side duration in a replayed graph, with no profiler
 * attached.  Same outputs as nlg_ternary_linear. */
int nlg_ternary_linear_timed(const float *x, const uint32_t *w2, const float *beta, float *y, uint32_t out,
                             uint32_t cols, unsigned long long *stamps, size_t stamps_bytes, void *stream);
size_t nlg_ternary_linear_timed_stamps(uint32_t out);

/* Tiled weight copies.  No counterpart in the reference, which reads the
 * row layout of ternary-rows (kernels.el:700-746) at every batch size; for
 * callers that run the batched linears above (4 or more tokens).
 * Registering 2-bit weights w2 [rows x cols/16] (cols a multiple of 256,
 * 16-byte aligned) makes a library-owned copy of them in the matrix-core
 * GEMM's load order (the same words; each wave then loads 1 KiB runs
 * instead of 32-byte pieces of 32 rows), which every linear given this w2
 * pointer with the same rows and cols at 4+ tokens reads instead.  The
 * copy is taken when this is called (it waits for `stream`).  Writes into
 * registered weights through this library -- nlg_upload, nlg_upload_file,
 * nlg_copy_d2d, nlg_zero, the repacks above -- refresh the copy in stream
 * order after the write (in place, so captured graphs see it); nlg_free of
 * the allocation holding w2 drops the registration.  Weights changed any
 * other way (a kernel of the caller's, a dispatch by name) need
 * nlg_ternary_tiled_register again, which refreshes the copy in place.
 * Results are bit-identical to the row layout's.  Costs rows (rounded up
 * to 32) x cols/4 bytes of device memory. */
int nlg_ternary_tiled_register(const uint32_t *w2, uint32_t rows, uint32_t cols, void *stream);
int nlg_ternary_tiled_unregister(const uint32_t *w2);

/* Synthetic data: n floats of sigma * N(0,1) from a counter-based
 * SplitMix64 stream (element 2p, 2p+1 = Box-Muller pair p); causal > 0 treats
 * the data as [.. x causal x causal] score tiles and writes -inf above each
 * tile's diagonal (the config-3 softmax input). */
int nlg_fill_normal(float *dev, uint64_t n, uint64_t seed, float sigma, uint32_t causal, void *stream);

/* ------------------------------------------------------------------------
 * A random-initialised ternary decoder stack (pre-norm, SwiGLU, GQA, RoPE,
 * fp16 KV cache, ternary LM head, greedy decode) built from the fusions
 * above.  The reference composes its models in Lisp over vkserver (the
 * nl-llm-* callers, not part of the reference tree); this is the same
 * composition run as one captured graph per token.
 * ---------------------------------------------------------------------- */
typedef struct nlg_stack nlg_stack;
typedef struct {
  uint32_t layers, d_model, heads, kv_heads, head_dim, d_ff, vocab, max_seq, batch;
  float rms_eps, rope_theta;
  uint64_t seed;
} nlg_stack_config;

/* Allocate and generate every weight on the device from cfg->seed. */
int nlg_stack_create(const nlg_stack_config *cfg, nlg_stack **out);
void nlg_stack_destroy(nlg_stack *s);
/* Begin `batch` sequences with prompts [batch x n_prompt] (host int32). */
int nlg_stack_start(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt);
/* Begin `batch` sequences and run every prompt token through the stack at
 * once (batch x n_prompt rows through the batched linears, causal attention
 * over the cache), then the LM head on each sequence's last prompt token:
 * the state is then that of nlg_stack_start + n_prompt steps (position
 * n_prompt, the first greedy token chosen), except that greedy choices are
 * kept only for the last prompt position.  batch x n_prompt <= 65535. */
int nlg_stack_prefill(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt);
/* Run `steps` token steps: the token at the current position goes through
 * every layer, its K/V are cached, and the next token is the prompt's while
 * the prompt lasts, else the greedy choice.  use_graph != 0 replays one
 * captured graph per step. */
int nlg_stack_step(nlg_stack *s, uint32_t steps, int use_graph);
/* One eager token step, as nlg_stack_step(s, 1, 0), that also returns the
 * residual stream it went through: xs (host) receives [layers + 1][batch]
 * [d_model] f32, the embedded token before layer 0 and the stream after
 * each layer.  For checking a layer at a time against a reference
 * composition; the reference has no counterpart (its model code runs the
 * named kernels from Lisp and can read any buffer back). */
int nlg_stack_step_trace(nlg_stack *s, float *xs);
/* nlg_stack_prefill that also writes the prompt rows' residual stream to xs
 * (host, [layers + 1][batch x n_prompt][d_model]: the embedded prompt rows,
 * then the rows after each layer; row z = sequence z / n_prompt, position
 * z % n_prompt), so that each layer of a prefill can be checked on its own
 * against the reference kernels (kernels.el:934-990, :340-365, :1249-1265). */
int nlg_stack_prefill_trace(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt, float *xs);
/* Current position (tokens consumed per sequence). */
int nlg_stack_position(nlg_stack *s, uint32_t *pos);
/* Token history [batch x max_seq] (prompt, then generated; -1 unwritten) and
 * greedy choices [batch x max_seq] (argmax after position p). */
int nlg_stack_tokens(nlg_stack *s, int32_t *tokens, int32_t *greedy);
/* Logits of the last step, [batch x vocab] (host). */
int nlg_stack_logits(nlg_stack *s, float *logits);
/* Device pointer and size of a named tensor ("wqkv", "bqkv", "wo", "bo",
 * "wgu", "bgu", "wd", "bd", "gattn", "gffn", "kc", "vc" with a layer;
 * "wlm", "blm", "gfinal", "emb", "rope_cos", "rope_sin", "x" with layer -1).
 * The tensors may be written.  The matrix-core linears (4+ rows) of a stack
 * read tiled copies of the 2-bit weights (wqkv, wo, wgu, wd, wlm); handing
 * out one of those pointers makes the next prefill / step / step trace
 * refresh the copies from the weights first, so weights written between
 * this call and that one are what every path computes with.  To write them
 * again after a step, ask for the pointer again. */
int nlg_stack_tensor(nlg_stack *s, const char *name, int layer, void **ptr, size_t *bytes);

#ifdef __cplusplus
}
#endif

#endif /* NLGPU_H */
