// nlg_dispatch.hip -- kernel names to launchers.
//
// Replaces get_kernel (host/vkserver.c:247-272), which loaded
// <kdir>/<name>.spv on first use and cached a pipeline by name.  Here the
// table is static: each name of lisp/nelisp-gpu-kernels.el on the hot path
// maps to a hand-written gfx950 kernel, with the binding count (:buffers)
// and push-constant count (:push) that name has in the reference.
#include <stdio.h>
#include <string.h>

#include "nlg_internal.h"

struct KEntry {
  const char *name;
  uint32_t nbuf, npush;
  nlg_launcher fn;
};

// Binding and push-constant counts are those of the cited DSL entry.
static const KEntry kTable[] = {
    {"vadd", 3, 1, L_vadd},                             // kernels.el:12
    {"matmul", 3, 3, L_matmul},                         // :17
    {"softmax", 2, 2, L_softmax},                       // :28
    {"linear", 4, 3, L_linear},                         // :71
    {"matmul-tiled", 3, 3, L_matmul_tiled},             // :82
    {"matmul-reg", 3, 3, L_matmul_reg},                 // :129
    {"scale", 3, 1, L_scale},                           // :141
    {"causal-mask", 1, 1, L_causal_mask},               // :148
    {"silu-mul", 3, 1, L_silu_mul},                     // :187
    {"attn-scores", 3, 4, L_attn_scores},               // :208
    {"attn-context", 3, 4, L_attn_context},             // :224
    {"decode-rope", 6, 2, L_decode_rope},               // :294
    {"cache-append", 3, 1, L_cache_append},             // :308
    {"decode-attn", 5, 3, L_decode_attn},               // :317
    {"decode-rope-b", 6, 3, L_decode_rope_b},           // :342
    {"cache-append-b", 3, 3, L_cache_append_b},         // :358
    {"decode-attn-b", 5, 5, L_decode_attn_b},           // :368
    {"quant-act", 2, 2, L_quant_act},                   // :529
    {"dp4a-dot", 5, 1, L_dp4a_dot},                     // :592
    {"bitlinear-dp4a", 8, 3, L_bitlinear_dp4a},         // :606
    {"bitlinear-dp4a-1f", 6, 3, L_bitlinear_dp4a_1f},   // :623
    {"bitlinear-dp4a-rows", 6, 3, L_bitlinear_dp4a_rows},  // :642
    {"ternary-rows", 5, 5, L_ternary_rows},             // :713
    {"add2", 3, 1, L_add2},                             // :816
    {"rmsnorm-heads", 3, 3, L_rmsnorm_heads},           // :828
    {"rope-half", 2, 5, L_rope_half},                   // :857
    {"pack-act-rows", 3, 3, L_pack_act_rows},           // :898
    {"attn-causal-gqa", 4, 4, L_attn_causal_gqa},       // :949
    {"bitlinear-packed", 5, 5, L_bitlinear_packed},     // :998
    {"bitlinear-packed-v", 5, 5, L_bitlinear_packed_v}, // :1022
    {"qkv-append", 3, 3, L_qkv_append},                 // :1044
    {"rmsnorm-istd", 2, 2, L_rmsnorm_istd},             // :1250
    {"rmsnorm-fwd", 4, 2, L_rmsnorm_fwd},               // :1259
    {"rope-apply", 5, 3, L_rope_apply},                 // :1290
    {"silu", 2, 1, L_silu},                             // :1306
    {"mul", 3, 1, L_mul},                               // :1322
    {"embed-gather", 3, 2, L_embed_gather},             // :1385
    // transposed linears (input gradients)
    {"ternary-rows-t", 4, 5, L_ternary_rows_t},         // :750
    {"dp4a-rows-t", 4, 4, L_dp4a_rows_t},               // :791
    // long-context decode (StreamingLLM ring, paged KV)
    {"cache-append-ring", 3, 3, L_cache_append_ring},   // :396
    {"decode-attn-stream", 7, 5, L_decode_attn_stream}, // :409
    {"attn-stream-entries", 7, 5, L_attn_stream_entries}, // :1056
    {"cache-append-paged", 4, 4, L_cache_append_paged}, // :1099
    {"decode-attn-paged", 6, 6, L_decode_attn_paged},   // :1112
    {"block-copy", 1, 4, L_block_copy},                 // :1184
    {"decode-rope-b-v", 6, 3, L_decode_rope_b_v},       // :1197
    {"cache-append-paged-v", 4, 4, L_cache_append_paged_v}, // :1212
    {"decode-attn-paged-v", 6, 6, L_decode_attn_paged_v},   // :1224
    // extension, no reference counterpart: 2-bit weights x pack-act-rows
    // activations, int32 accumulation (see nlg_ternary_linear_i8)
    {"ternary-i8", 6, 3, L_ternary_i8},
};
static const int kCount = (int)(sizeof kTable / sizeof kTable[0]);

static const KEntry *find(const char *name) {
  if (!name) return nullptr;
  for (int i = 0; i < kCount; i++)
    if (!strcmp(kTable[i].name, name)) return &kTable[i];
  return nullptr;
}

int nlg_need(const nlg_buffer *b, int i, uint64_t need, const char *kname) {
  if ((uint64_t)b[i].nfloats < need)
    return nlg_fail("%s: buffer %d holds %u elements, needs %llu", kname, i, b[i].nfloats,
                    (unsigned long long)need);
  if (need && !b[i].ptr) return nlg_fail("%s: buffer %d is null", kname, i);
  return NLG_OK;
}

extern "C" int nlg_kernel_count(void) { return kCount; }
extern "C" const char *nlg_kernel_name(int i) { return (i >= 0 && i < kCount) ? kTable[i].name : nullptr; }
extern "C" int nlg_kernel_lookup(const char *name) {
  const KEntry *e = find(name);
  return e ? (int)(e - kTable) : -1;
}
extern "C" int nlg_kernel_abi(const char *name, uint32_t *nbuf, uint32_t *npush) {
  const KEntry *e = find(name);
  if (!e) return nlg_fail("no kernel named '%s'", name ? name : "(null)");
  if (nbuf) *nbuf = e->nbuf;
  if (npush) *npush = e->npush;
  return NLG_OK;
}

extern "C" int nlg_dispatch(const char *name, const nlg_buffer *bufs, uint32_t nbuf,
                            const uint32_t *push, uint32_t npush, uint32_t groups, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  const KEntry *e = find(name);
  if (!e) return nlg_fail("no kernel named '%s'", name ? name : "(null)");
  if (nbuf != e->nbuf)
    return nlg_fail("%s: %u buffers bound, the kernel has %u", e->name, nbuf, e->nbuf);
  // The reference pipeline layout takes npush from the first call; a
  // shader reading more constants than were pushed reads undefined values.
  // Require at least the kernel's count; extra constants are ignored.
  if (npush < e->npush)
    return nlg_fail("%s: %u push constants, the kernel reads %u", e->name, npush, e->npush);
  uint32_t p[16] = {0};
  for (uint32_t i = 0; i < npush && i < 16; i++) p[i] = push[i];
  return e->fn(bufs, p, groups, nlg_stream(stream));
}
