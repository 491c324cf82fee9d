// nlg_stack.hip -- a random-initialised ternary decoder stack run from the
// decoder-layer fusions, one captured graph per token.
//
// Per token step (every sequence of the batch at the same position, as
// decode-attn-b assumes, kernels.el:366-390):
//   for each layer:
//     q, K[pos], V[pos] = RoPE(linear_qkv(rmsnorm(x)))   nlg_rms_ternary_qkv_rope
//     a = attention(q, K[0..pos], V[0..pos])             nlg_decode_attn_f16
//     x = x + linear_o(a)                                nlg_ternary_linear_residual
//     h = silu(gate) * up, [gate|up] = linear(rmsnorm(x)) nlg_rms_ternary_swiglu
//     x = x + linear_down(h)                             nlg_ternary_linear_residual
//   logits = linear_lm(rmsnorm(x)); next token; x = embedding(next)
// Every linear is 2-bit ternary with int8 absmax activations and one fp32
// scale per output row.  Position, prompt and token history live on the
// device, so one captured step replays unchanged for every token.
//
// Weights are drawn on the device from a counter-based SplitMix64 stream
// (element i of a tensor uses output i+1 of the stream seeded with that
// tensor's seed): trits -1/0/+1 with probabilities 1/4, 1/2, 1/4; gains
// uniform in [0.75, 1.25); embeddings N(0,1) by Box-Muller on pairs.  The
// scale of a linear with `cols` inputs is 1/sqrt(cols/2), which keeps unit
// RMS through it (a trit has variance 1/2).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "nlg_internal.h"

// ------------------------------------------------------------ generators

__device__ __forceinline__ uint64_t sm64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ double sm_uniform(uint64_t seed, uint64_t i) {
  return (double)(sm64(seed, i) >> 11) * (1.0 / 9007199254740992.0);
}

// Packed trits for logical rows [0, rows) of a [rows x cols] tensor, stored
// at physical row r*mult + off (mult 2 interleaves gate and up).
__global__ void k_gen_trits(uint32_t *w2, uint32_t rows, uint32_t cols, uint64_t seed, uint32_t mult,
                            uint32_t off) {
  const uint32_t wng = (cols + 15) / 16;
  const uint64_t n = (uint64_t)rows * wng;
  for (uint64_t idx = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; idx < n;
       idx += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t r = idx / wng, wd = idx % wng;
    uint32_t word = 0;
    for (uint32_t f = 0; f < 16; f++) {
      const uint64_t c = wd * 16 + f;
      if (c >= cols) break;
      const double u = sm_uniform(seed, r * cols + c);
      const uint32_t code = u < 0.25 ? 3u : (u < 0.75 ? 0u : 1u);  // -1, 0, +1
      word |= code << (2 * f);
    }
    w2[(r * mult + off) * wng + wd] = word;
  }
}

__global__ void k_gen_uniform(float *dst, uint64_t n, uint64_t seed, double lo, double hi) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = (float)(lo + (hi - lo) * sm_uniform(seed, i));
}

// Element 2p and 2p+1 share the pair (u1 = 1 - u(2p), u2 = u(2p+1)):
// r cos(2 pi u2) and r sin(2 pi u2), r = sqrt(-2 ln u1).
// sigma * that; with causal > 0 the data is [.. x causal x causal] score
// tiles and entries with column > row are -inf.
__global__ void k_gen_normal(float *dst, uint64_t n, uint64_t seed, float sigma, uint32_t causal) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t p = i >> 1;
    const double u1 = 1.0 - sm_uniform(seed, 2 * p), u2 = sm_uniform(seed, 2 * p + 1);
    const double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
    float v = (float)(r * ((i & 1) ? sin(t) : cos(t)));
    if (sigma != 1.0f) v = v * sigma;
    if (causal && (i % causal) > (i / causal) % causal) v = -INFINITY;
    dst[i] = v;
  }
}

extern "C" int nlg_fill_normal(float *dev, uint64_t n, uint64_t seed, float sigma, uint32_t causal,
                               void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!n) return NLG_OK;
  const uint64_t g = n / 256 + 1 < 65536 ? n / 256 + 1 : 65536;
  hipLaunchKernelGGL(k_gen_normal, dim3((uint32_t)g), dim3(256), 0, nlg_stream(stream), dev, n, seed, sigma,
                     causal);
  NLG_LAUNCHED("fill normal");
  return NLG_OK;
}

__global__ void k_fill_f32(float *dst, uint64_t n, float v) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = v;
}

// x[b] = emb[tok[b * tstride]]; tokens are validated before they get here.
__global__ void k_embed_rows(const float *emb, const int32_t *tok, uint32_t tstride, float *x,
                             uint32_t dim) {
  const uint32_t b = blockIdx.y;
  const int32_t t = tok[(size_t)b * tstride];
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < dim; j += gridDim.x * blockDim.x)
    x[(size_t)b * dim + j] = emb[(size_t)t * dim + j];
}

// ------------------------------------------------------------ sampling

__device__ __forceinline__ bool better(float v, int32_t i, float bv, int32_t bi) {
  if (i < 0) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

struct SampleArgs {
  const float *pval;
  const int32_t *pidx;
  uint32_t nparts;           // per sequence
  const int32_t *prompt;     // [B x max_seq]
  int32_t *hist, *greedy;    // [B x max_seq]
  int32_t *pos;
  const int32_t *plen;
  const float *emb;
  float *x;                  // [B x dim]
  uint32_t dim, batch, max_seq, vocab;
};

// The greedy token after position p of one sequence (ONE: the only one,
// and this workgroup then advances the position; otherwise sequence
// blockIdx.x, and k_advance moves the position once every row is done); the
// next token is the prompt's while it lasts; its embedding becomes x.
template <bool ONE>
__global__ __launch_bounds__(1024) void k_sample(SampleArgs a) {
  __shared__ float sv[16];
  __shared__ int32_t si[16];
  __shared__ int32_t s_tok;
  const int32_t p = a.pos[0];
  const int32_t plen = a.plen[0];
  const int nw = blockDim.x >> 6, w = threadIdx.x >> 6;
  const uint32_t b = ONE ? 0u : blockIdx.x;
  const float *pv = a.pval + (size_t)b * a.nparts;
  const int32_t *pi = a.pidx + (size_t)b * a.nparts;
  float v = -INFINITY;
  int32_t i = -1;
  // eight partials per thread in flight at a time (independent loads)
  for (uint32_t j0 = threadIdx.x; j0 < a.nparts; j0 += 8 * blockDim.x) {
    float ov[8];
    int32_t oi[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const uint32_t j = j0 + u * blockDim.x;
      const uint32_t jc = j < a.nparts ? j : a.nparts - 1;
      ov[u] = pv[jc];
      oi[u] = j < a.nparts ? pi[jc] : -1;
    }
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (better(ov[u], oi[u], v, i)) { v = ov[u]; i = oi[u]; }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int32_t oi = __shfl_xor(i, off);
    if (better(ov, oi, v, i)) { v = ov; i = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = sv[0]; i = si[0];
    for (int k = 1; k < nw; k++)
      if (better(sv[k], si[k], v, i)) { v = sv[k]; i = si[k]; }
    const size_t row = (size_t)b * a.max_seq;
    int32_t t = i < 0 ? 0 : i;
    if (p + 1 < plen) t = a.prompt[row + p + 1];
    if (t < 0 || (uint32_t)t >= a.vocab) t = 0;
    if (p >= 0 && (uint32_t)p < a.max_seq) a.greedy[row + p] = i;
    if (p + 1 >= 0 && (uint32_t)(p + 1) < a.max_seq) a.hist[row + p + 1] = t;
    s_tok = t;
  }
  __syncthreads();
  const int32_t t = s_tok;
  for (uint32_t j = threadIdx.x; j < a.dim; j += blockDim.x)
    a.x[(size_t)b * a.dim + j] = a.emb[(size_t)t * a.dim + j];
  if (ONE && threadIdx.x == 0) a.pos[0] = p + 1;  // every thread read p before the barrier
}

__global__ void k_advance(int32_t *pos) {
  if (threadIdx.x == 0) pos[0] = pos[0] + 1;
}

// ------------------------------------------------------------ the stack

struct Layer {
  uint32_t *wqkv, *wo, *wgu, *wd;
  float *bqkv, *bo, *bgu, *bd, *gattn, *gffn;
  uint16_t *kc, *vc;
};

struct nlg_stack {
  nlg_stack_config c;
  uint32_t nq, nkv;
  std::vector<Layer> L;
  uint32_t *wlm;
  float *blm, *gfinal, *emb, *co, *si;
  float *x, *q, *att, *h, *logits, *pval;
  int32_t *pidx, *pos, *plen, *prompt, *hist, *greedy;
  uint32_t nparts;
  void *attn_ws;
  size_t attn_ws_bytes;
  bool attn_fused;  // merge folded into the output projection
  std::vector<void *> allocs;
  // prefill rows (batch x prompt tokens), allocated at the first prefill
  float *px, *pq, *ph;
  void *pattn_ws;
  size_t pattn_ws_bytes;
  uint32_t pcap;
  bool tiled;  // prompt-order copies of the layer weights registered
  // a weight pointer was handed out (nlg_stack_tensor): the next prefill or
  // step refreshes the tiled copies from the row layout first
  bool retile;
  void *graph;
  uint32_t host_pos;
  bool started;
};

static void *salloc(nlg_stack *s, size_t bytes) {
  void *p = nlg_malloc(bytes ? bytes : 4);
  if (p) s->allocs.push_back(p);
  return p;
}

static uint64_t tensor_seed(uint64_t seed, uint32_t layer, uint32_t tensor) {
  return seed + 1000003ull * (layer + 1) + tensor;
}

static int gen_grid(uint64_t n) { return (int)(n / 256 + 1 < 65536 ? n / 256 + 1 : 65536); }

static int gen_trits(uint32_t *w2, uint32_t rows, uint32_t cols, uint64_t seed, uint32_t mult,
                     uint32_t off) {
  const uint64_t n = (uint64_t)rows * ((cols + 15) / 16);
  hipLaunchKernelGGL(k_gen_trits, dim3(gen_grid(n)), dim3(256), 0, nlg_stream(nullptr), w2, rows, cols,
                     seed, mult, off);
  NLG_LAUNCHED("generate trits");
  return NLG_OK;
}
static int fill(float *d, uint64_t n, float v) {
  hipLaunchKernelGGL(k_fill_f32, dim3(gen_grid(n)), dim3(256), 0, nlg_stream(nullptr), d, n, v);
  NLG_LAUNCHED("fill");
  return NLG_OK;
}
static int gen_uniform(float *d, uint64_t n, uint64_t seed, double lo, double hi) {
  hipLaunchKernelGGL(k_gen_uniform, dim3(gen_grid(n)), dim3(256), 0, nlg_stream(nullptr), d, n, seed, lo, hi);
  NLG_LAUNCHED("generate uniform");
  return NLG_OK;
}
static int gen_normal(float *d, uint64_t n, uint64_t seed) {
  hipLaunchKernelGGL(k_gen_normal, dim3(gen_grid(n)), dim3(256), 0, nlg_stream(nullptr), d, n, seed, 1.0f, 0u);
  NLG_LAUNCHED("generate normal");
  return NLG_OK;
}

extern "C" void nlg_stack_destroy(nlg_stack *s) {
  if (!s) return;
  if (s->graph) nlg_graph_destroy(s->graph);
  if (s->tiled)
    for (Layer &y : s->L)
      for (const uint32_t *w : {y.wqkv, y.wo, y.wgu, y.wd}) (void)nlg_ternary_tiled_unregister(w);
  if (s->tiled) (void)nlg_ternary_tiled_unregister(s->wlm);
  for (void *p : s->allocs) nlg_free(p);
  for (void *p : {(void *)s->px, (void *)s->pq, (void *)s->ph, s->pattn_ws})
    if (p) nlg_free(p);
  delete s;
}

static int stack_alloc(nlg_stack *s) {
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, f = c.d_ff, B = c.batch;
  const uint32_t qkv = s->nq + 2 * s->nkv;
  const size_t cache = (size_t)B * c.kv_heads * c.max_seq * c.head_dim * 2;
  s->L.resize(c.layers);
  for (uint32_t l = 0; l < c.layers; l++) {
    Layer &y = s->L[l];
    y.wqkv = (uint32_t *)salloc(s, (size_t)qkv * (d / 16) * 4);
    y.wo = (uint32_t *)salloc(s, (size_t)d * (s->nq / 16) * 4);
    y.wgu = (uint32_t *)salloc(s, (size_t)2 * f * (d / 16) * 4);
    y.wd = (uint32_t *)salloc(s, (size_t)d * (f / 16) * 4);
    y.bqkv = (float *)salloc(s, (size_t)qkv * 4);
    y.bo = (float *)salloc(s, 4);
    y.bgu = (float *)salloc(s, (size_t)2 * f * 4);
    y.bd = (float *)salloc(s, 4);
    y.gattn = (float *)salloc(s, (size_t)d * 4);
    y.gffn = (float *)salloc(s, (size_t)d * 4);
    y.kc = (uint16_t *)salloc(s, cache);
    y.vc = (uint16_t *)salloc(s, cache);
    if (!y.wqkv || !y.wo || !y.wgu || !y.wd || !y.bqkv || !y.bo || !y.bgu || !y.bd || !y.gattn ||
        !y.gffn || !y.kc || !y.vc)
      return NLG_ERR;
  }
  s->wlm = (uint32_t *)salloc(s, (size_t)c.vocab * (d / 16) * 4);
  s->blm = (float *)salloc(s, 4);
  s->gfinal = (float *)salloc(s, (size_t)d * 4);
  s->emb = (float *)salloc(s, (size_t)c.vocab * d * 4);
  s->co = (float *)salloc(s, (size_t)c.max_seq * (c.head_dim / 2) * 4);
  s->si = (float *)salloc(s, (size_t)c.max_seq * (c.head_dim / 2) * 4);
  s->x = (float *)salloc(s, (size_t)B * d * 4);
  s->q = (float *)salloc(s, (size_t)B * s->nq * 4);
  s->att = (float *)salloc(s, (size_t)B * s->nq * 4);
  s->h = (float *)salloc(s, (size_t)B * f * 4);
  s->logits = (float *)salloc(s, (size_t)B * c.vocab * 4);
  s->nparts = nlg_argmax_parts(B, d, c.vocab);
  s->pval = (float *)salloc(s, (size_t)B * s->nparts * 4);
  s->pidx = (int32_t *)salloc(s, (size_t)B * s->nparts * 4);
  s->pos = (int32_t *)salloc(s, 4);
  s->plen = (int32_t *)salloc(s, 4);
  s->prompt = (int32_t *)salloc(s, (size_t)B * c.max_seq * 4);
  s->hist = (int32_t *)salloc(s, (size_t)B * c.max_seq * 4);
  s->greedy = (int32_t *)salloc(s, (size_t)B * c.max_seq * 4);
  s->attn_ws_bytes = nlg_decode_attn_f16_workspace(B, c.heads, c.kv_heads, c.head_dim, c.max_seq);
  s->attn_ws = salloc(s, s->attn_ws_bytes);
  s->attn_fused = nlg_attn_chunk_count(c.head_dim, c.max_seq) <= NLG_ATTN_MAX_CHUNKS;
  {  // reserve the batched linears' scratch now: it cannot grow under capture
    uint32_t widest = d > f ? d : f;
    widest = widest > s->nq ? widest : s->nq;
    if (!nlg_scratch(nlg_batched_scratch_bytes(B, widest), nlg_stream(nullptr))) return NLG_ERR;
  }
  if (!s->wlm || !s->blm || !s->gfinal || !s->emb || !s->co || !s->si || !s->x || !s->q || !s->att ||
      !s->h || !s->logits || !s->pval || !s->pidx || !s->pos || !s->plen || !s->prompt || !s->hist ||
      !s->greedy || !s->attn_ws)
    return NLG_ERR;
  return NLG_OK;
}

static int stack_generate(nlg_stack *s) {
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, f = c.d_ff;
  const float sd = (float)(1.0 / sqrt(0.5 * d)), sq = (float)(1.0 / sqrt(0.5 * s->nq)),
              sf = (float)(1.0 / sqrt(0.5 * f));
  for (uint32_t l = 0; l < c.layers; l++) {
    Layer &y = s->L[l];
    // tensors: 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down, 7 attn gain, 8 ffn gain
    if (gen_trits(y.wqkv, s->nq, d, tensor_seed(c.seed, l, 0), 1, 0) ||
        gen_trits(y.wqkv + (size_t)s->nq * (d / 16), s->nkv, d, tensor_seed(c.seed, l, 1), 1, 0) ||
        gen_trits(y.wqkv + (size_t)(s->nq + s->nkv) * (d / 16), s->nkv, d, tensor_seed(c.seed, l, 2), 1, 0) ||
        gen_trits(y.wo, d, s->nq, tensor_seed(c.seed, l, 3), 1, 0) ||
        gen_trits(y.wgu, f, d, tensor_seed(c.seed, l, 4), 2, 0) ||
        gen_trits(y.wgu, f, d, tensor_seed(c.seed, l, 5), 2, 1) ||
        gen_trits(y.wd, d, f, tensor_seed(c.seed, l, 6), 1, 0) ||
        fill(y.bqkv, s->nq + 2 * s->nkv, sd) || fill(y.bo, 1, sq) || fill(y.bgu, 2 * f, sd) ||
        fill(y.bd, 1, sf) || gen_uniform(y.gattn, d, tensor_seed(c.seed, l, 7), 0.75, 1.25) ||
        gen_uniform(y.gffn, d, tensor_seed(c.seed, l, 8), 0.75, 1.25))
      return NLG_ERR;
  }
  // 0 LM head, 1 final gain, 2 embedding
  if (gen_trits(s->wlm, c.vocab, d, tensor_seed(c.seed, c.layers, 0), 1, 0) || fill(s->blm, 1, sd) ||
      gen_uniform(s->gfinal, d, tensor_seed(c.seed, c.layers, 1), 0.75, 1.25) ||
      gen_normal(s->emb, (uint64_t)c.vocab * d, tensor_seed(c.seed, c.layers, 2)))
    return NLG_ERR;
  // RoPE tables: angle = p / theta^(2m/hd), in double, rounded to f32
  const uint32_t half = c.head_dim / 2;
  std::vector<float> co((size_t)c.max_seq * half), si((size_t)c.max_seq * half);
  for (uint32_t p = 0; p < c.max_seq; p++)
    for (uint32_t m = 0; m < half; m++) {
      const double ang = (double)p / pow((double)c.rope_theta, (2.0 * m) / c.head_dim);
      co[(size_t)p * half + m] = (float)cos(ang);
      si[(size_t)p * half + m] = (float)sin(ang);
    }
  if (nlg_upload(s->co, co.data(), co.size() * 4) || nlg_upload(s->si, si.data(), si.size() * 4))
    return NLG_ERR;
  NLG_HIP(hipStreamSynchronize(nlg_stream(nullptr)));
  return NLG_OK;
}

static int stack_tile(nlg_stack *s);

extern "C" int nlg_stack_create(const nlg_stack_config *cfg, nlg_stack **out) {
  if (!cfg || !out) return nlg_fail("stack: null argument");
  *out = nullptr;
  if (nlg_ensure_init()) return NLG_ERR;
  const nlg_stack_config &c = *cfg;
  if (!c.layers || !c.d_model || !c.heads || !c.kv_heads || !c.head_dim || !c.d_ff || !c.vocab ||
      !c.max_seq || !c.batch)
    return nlg_fail("stack: every size must be nonzero");
  if (c.heads % c.kv_heads) return nlg_fail("stack: heads must be a multiple of kv_heads");
  const uint32_t G = c.heads / c.kv_heads;
  if ((c.head_dim != 64 && c.head_dim != 128) || (G != 1 && G != 2 && G != 4 && G != 8))
    return nlg_fail("stack: head_dim must be 64 or 128 and heads/kv_heads 1, 2, 4 or 8");
  if (c.d_model % 64 || c.d_ff % 64 || (c.heads * c.head_dim) % 64 || c.d_model > 16384 ||
      c.d_ff > 16384 || c.heads * c.head_dim > 16384)
    return nlg_fail("stack: d_model, d_ff and heads*head_dim must be multiples of 64, at most 16384");
  if (c.vocab >= (1u << 31) || c.batch > 4096 || c.max_seq > (1u << 20))
    return nlg_fail("stack: vocab, batch or max_seq out of range");
  if (!(c.rms_eps >= 0.0f) || !(c.rope_theta > 0.0f)) return nlg_fail("stack: bad eps or theta");
  nlg_stack *s = new nlg_stack();
  s->c = c;
  s->nq = c.heads * c.head_dim;
  s->nkv = c.kv_heads * c.head_dim;
  if (stack_alloc(s) || stack_generate(s) || (c.batch >= NLG_BATCHED_MIN && stack_tile(s))) {
    nlg_stack_destroy(s);
    return NLG_ERR;
  }
  *out = s;
  return NLG_OK;
}

// Attention and its output projection: chunk pass, then the merge folded
// into the projection's prologue when the chunks fit it, else a separate
// merge launch.
static int stack_attention(nlg_stack *s, Layer &y) {
  const nlg_stack_config &c = s->c;
  const uint32_t B = c.batch, d = c.d_model;
  if (s->attn_fused)
    return nlg_decode_attn_f16_chunks(s->q, y.kc, y.vc, s->pos, B, c.heads, c.kv_heads, c.head_dim, c.max_seq,
                                      s->attn_ws, s->attn_ws_bytes, nullptr) ||
           nlg_attn_ternary_linear_residual(s->attn_ws, s->attn_ws_bytes, B, c.heads, c.kv_heads, c.head_dim,
                                            c.max_seq, y.wo, nullptr, y.bo, 0, s->x, s->x, d, nullptr);
  return nlg_decode_attn_f16(s->q, y.kc, y.vc, s->pos, s->att, B, c.heads, c.kv_heads, c.head_dim, c.max_seq,
                             s->attn_ws, s->attn_ws_bytes, nullptr) ||
         nlg_ternary_linear_residual(s->att, y.wo, nullptr, y.bo, 0, s->x, s->x, B, d, s->nq, nullptr);
}

static int stack_head(nlg_stack *s);

// The matrix-core GEMMs (4+ rows: prompts, and every step at batch >= 4)
// read tiled copies of the layer weights, and of the LM head when it runs
// on 4+ rows (batch >= 4): one more copy of them, made once.
// Registering again refreshes a copy in place (same buffers: the captured
// step graph keeps reading them).
static int stack_tile(nlg_stack *s) {
  if (s->tiled && !s->retile) return NLG_OK;
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, f = c.d_ff, qkv = s->nq + 2 * s->nkv;
  s->tiled = true;
  s->retile = false;
  for (Layer &y : s->L) {
    if ((d % 256 == 0 && (nlg_ternary_tiled_register(y.wqkv, qkv, d, nullptr) ||
                          nlg_ternary_tiled_register(y.wgu, 2 * f, d, nullptr))) ||
        (s->nq % 256 == 0 && nlg_ternary_tiled_register(y.wo, d, s->nq, nullptr)) ||
        (f % 256 == 0 && nlg_ternary_tiled_register(y.wd, d, f, nullptr)))
      return NLG_ERR;
  }
  if (c.batch >= NLG_BATCHED_MIN && d % 256 == 0 && nlg_ternary_tiled_register(s->wlm, c.vocab, d, nullptr))
    return NLG_ERR;
  return NLG_OK;
}
static int upload_prompt(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt, bool all_hist);

// One token step for the whole batch, enqueued on the library stream.
// trace (device, may be null) receives the residual stream before layer 0
// and after every layer, [layers + 1][batch][d_model].
static int stack_enqueue(nlg_stack *s, float *trace = nullptr) {
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, f = c.d_ff, B = c.batch;
  const size_t xbytes = (size_t)B * d * 4;
  if (trace && nlg_copy_d2d(trace, s->x, xbytes, nullptr)) return NLG_ERR;
  for (uint32_t l = 0; l < c.layers; l++) {
    Layer &y = s->L[l];
    if (nlg_rms_ternary_qkv_rope(s->x, y.gattn, c.rms_eps, y.wqkv, y.bqkv, 1, s->q, y.kc, y.vc, s->co,
                                 s->si, s->pos, B, c.heads, c.kv_heads, c.head_dim, c.max_seq, d,
                                 nullptr) ||
        stack_attention(s, y) ||
        nlg_rms_ternary_swiglu(s->x, y.gffn, c.rms_eps, y.wgu, y.bgu, 1, s->h, B, f, d, nullptr) ||
        nlg_ternary_linear_residual(s->h, y.wd, nullptr, y.bd, 0, s->x, s->x, B, d, f, nullptr))
      return NLG_ERR;
    if (trace && nlg_copy_d2d(trace + (size_t)(l + 1) * B * d, s->x, xbytes, nullptr)) return NLG_ERR;
  }
  return stack_head(s);
}

// Final norm, LM head with the greedy partials, then the next token.
static int stack_head(nlg_stack *s) {
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, B = c.batch;
  FusedArgs a{};
  a.x = s->x; a.gain = s->gfinal; a.eps = c.rms_eps; a.w2 = s->wlm; a.beta = s->blm;
  a.seq = B; a.out = c.vocab; a.cols = d; a.y = s->logits; a.ystride = c.vocab;
  a.pval = s->pval; a.pidx = s->pidx;
  const int rpw = nlg_fused_rows_per_wave(c.vocab, NLG_EPI_ARGMAX, d);
  if (nlg_fused_launch(a, NLG_PRO_RMS, NLG_EPI_ARGMAX, rpw, nlg_stream(nullptr))) return NLG_ERR;
  SampleArgs sa;
  sa.pval = s->pval; sa.pidx = s->pidx; sa.nparts = s->nparts; sa.prompt = s->prompt;
  sa.hist = s->hist; sa.greedy = s->greedy; sa.pos = s->pos; sa.plen = s->plen; sa.emb = s->emb;
  sa.x = s->x; sa.dim = d; sa.batch = B; sa.max_seq = c.max_seq; sa.vocab = c.vocab;
  if (B == 1) {
    hipLaunchKernelGGL(k_sample<true>, dim3(1), dim3(1024), 0, nlg_stream(nullptr), sa);
  } else {
    hipLaunchKernelGGL(k_sample<false>, dim3(B), dim3(1024), 0, nlg_stream(nullptr), sa);
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, nlg_stream(nullptr), s->pos);
  }
  NLG_LAUNCHED("sample");
  return NLG_OK;
}

extern "C" int nlg_stack_start(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt) {
  if (!s || !prompts) return nlg_fail("stack start: null argument");
  const nlg_stack_config &c = s->c;
  if (upload_prompt(s, prompts, n_prompt, false)) return NLG_ERR;
  hipLaunchKernelGGL(k_embed_rows, dim3(nlg_blocks(c.d_model, 256), c.batch), dim3(256), 0,
                     nlg_stream(nullptr), s->emb, s->prompt, c.max_seq, s->x, c.d_model);
  NLG_LAUNCHED("embed");
  NLG_HIP(hipStreamSynchronize(nlg_stream(nullptr)));
  s->host_pos = 0;
  s->started = true;
  return NLG_OK;
}

// Prefill rows: row z = sequence z / P, prompt position z % P.
__global__ void k_embed_prompt(const float *emb, const int32_t *prompt, uint32_t max_seq, uint32_t P,
                               float *x, uint32_t dim) {
  const uint32_t z = blockIdx.y, b = z / P, t = z % P;
  const int32_t tok = prompt[(size_t)b * max_seq + t];
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < dim; j += gridDim.x * blockDim.x)
    x[(size_t)z * dim + j] = emb[(size_t)tok * dim + j];
}
__global__ void k_last_rows(const float *px, uint32_t P, float *x, uint32_t dim) {
  const uint32_t b = blockIdx.y;
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < dim; j += gridDim.x * blockDim.x)
    x[(size_t)b * dim + j] = px[((size_t)b * P + P - 1) * dim + j];
}

static int upload_prompt(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt, bool all_hist) {
  const nlg_stack_config &c = s->c;
  if (!n_prompt || n_prompt > c.max_seq) return nlg_fail("stack: prompt length must be 1..max_seq");
  std::vector<int32_t> pr((size_t)c.batch * c.max_seq, 0), hist((size_t)c.batch * c.max_seq, -1);
  for (uint32_t b = 0; b < c.batch; b++)
    for (uint32_t i = 0; i < n_prompt; i++) {
      const int32_t t = prompts[(size_t)b * n_prompt + i];
      if (t < 0 || (uint32_t)t >= c.vocab) return nlg_fail("stack: token %d out of range", t);
      pr[(size_t)b * c.max_seq + i] = t;
      if (all_hist || i == 0) hist[(size_t)b * c.max_seq + i] = t;
    }
  const int32_t zero = 0, plen = (int32_t)n_prompt;
  if (nlg_upload(s->prompt, pr.data(), pr.size() * 4) || nlg_upload(s->hist, hist.data(), hist.size() * 4) ||
      nlg_upload(s->greedy, std::vector<int32_t>(hist.size(), -1).data(), hist.size() * 4) ||
      nlg_upload(s->pos, &zero, 4) || nlg_upload(s->plen, &plen, 4))
    return NLG_ERR;
  return NLG_OK;
}

// trace (device, may be null): the prompt rows' residual stream before
// layer 0 and after every layer, [layers + 1][batch x n_prompt][d_model].
static int stack_prefill(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt, float *trace) {
  if (!s || !prompts) return nlg_fail("stack prefill: null argument");
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, f = c.d_ff, B = c.batch, P = n_prompt;
  if (upload_prompt(s, prompts, n_prompt, true)) return NLG_ERR;
  const uint64_t T64 = (uint64_t)B * P;
  if (T64 > 65535) return nlg_fail("stack prefill: batch x prompt = %llu rows > 65535", (unsigned long long)T64);
  const uint32_t T = (uint32_t)T64;
  hipStream_t st = nlg_stream(nullptr);
  if (T > s->pcap) {  // grow the prefill rows (eager, outside any capture)
    NLG_HIP(hipStreamSynchronize(st));
    for (void *p : {(void *)s->px, (void *)s->pq, (void *)s->ph, s->pattn_ws})
      if (p) nlg_free(p);
    s->px = (float *)nlg_malloc((size_t)T * d * 4);
    s->pq = (float *)nlg_malloc((size_t)T * s->nq * 4);
    s->ph = (float *)nlg_malloc((size_t)T * f * 4);
    s->pattn_ws_bytes = (size_t)T * s->nq * 4;
    s->pattn_ws = nlg_malloc(s->pattn_ws_bytes);
    if (!s->px || !s->pq || !s->ph || !s->pattn_ws) return NLG_ERR;
    s->pcap = T;
  }
  if ((T >= NLG_BATCHED_MIN || s->tiled) && stack_tile(s)) return NLG_ERR;
  hipLaunchKernelGGL(k_embed_prompt, dim3(nlg_blocks(d, 256), T), dim3(256), 0, st, s->emb, s->prompt,
                     c.max_seq, P, s->px, d);
  NLG_LAUNCHED("embed prompt");
  const size_t rows_bytes = (size_t)T * d * 4;
  if (trace) NLG_HIP(hipMemcpyAsync(trace, s->px, rows_bytes, hipMemcpyDeviceToDevice, st));
  float *pctx = (float *)s->pattn_ws;  // [T][nq] attention output
  for (uint32_t l = 0; l < c.layers; l++) {
    Layer &y = s->L[l];
    FusedArgs q{};
    q.x = s->px; q.gain = y.gattn; q.eps = c.rms_eps; q.w2 = y.wqkv; q.beta = y.bqkv; q.beta_per_row = 1;
    q.seq = T; q.nq = s->nq; q.nkv = s->nkv; q.out = s->nq + 2 * s->nkv; q.cols = d; q.y = s->pq;
    q.ystride = s->nq; q.hd = c.head_dim; q.kvheads = c.kv_heads; q.max_seq = c.max_seq; q.co = s->co;
    q.si = s->si; q.pos = s->pos; q.kc = y.kc; q.vc = y.vc; q.qper = P;
    if (nlg_fused_launch(q, NLG_PRO_RMS, NLG_EPI_QKV, 0, st)) return NLG_ERR;
    // prompt attention and the output projection (a split attention
    // leaves the merged context quantised for it); prompts start at
    // position 0, so no row attends past P
    if (nlg_prefill_attn_o_resid(s->pq, y.kc, y.vc, s->pos, T, P, c.heads, c.kv_heads, c.head_dim, c.max_seq, P,
                                 pctx, y.wo, nullptr, y.bo, 0, s->px, s->px, d, st))
      return NLG_ERR;
    FusedArgs g{};
    g.x = s->px; g.gain = y.gffn; g.eps = c.rms_eps; g.w2 = y.wgu; g.beta = y.bgu; g.beta_per_row = 1;
    g.seq = T; g.out = 2 * f; g.cols = d; g.y = s->ph; g.ystride = f;
    if (nlg_fused_launch(g, NLG_PRO_RMS, NLG_EPI_SWIGLU, 0, st)) return NLG_ERR;
    FusedArgs w{};
    w.x = s->ph; w.w2 = y.wd; w.beta = y.bd; w.seq = T; w.out = d; w.cols = f; w.y = s->px; w.ystride = d;
    w.res = s->px; w.rstride = d;
    if (nlg_fused_launch(w, NLG_PRO_NONE, NLG_EPI_RESID, 0, st)) return NLG_ERR;
    if (trace)
      NLG_HIP(hipMemcpyAsync((char *)trace + (size_t)(l + 1) * rows_bytes, s->px, rows_bytes, hipMemcpyDeviceToDevice, st));
  }
  hipLaunchKernelGGL(k_last_rows, dim3(nlg_blocks(d, 256), B), dim3(256), 0, st, s->px, P, s->x, d);
  NLG_LAUNCHED("last prompt rows");
  const int32_t last = (int32_t)P - 1;
  NLG_HIP(hipMemcpyAsync(s->pos, &last, 4, hipMemcpyHostToDevice, st));
  if (stack_head(s)) return NLG_ERR;
  NLG_HIP(hipStreamSynchronize(st));
  s->host_pos = P;
  s->started = true;
  return NLG_OK;
}

extern "C" int nlg_stack_prefill(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt) {
  return stack_prefill(s, prompts, n_prompt, nullptr);
}

extern "C" int nlg_stack_prefill_trace(nlg_stack *s, const int32_t *prompts, uint32_t n_prompt, float *xs) {
  if (!s || !prompts || !xs) return nlg_fail("stack prefill trace: null argument");
  if (!n_prompt || n_prompt > s->c.max_seq) return nlg_fail("stack: prompt length must be 1..max_seq");
  const size_t bytes = (size_t)(s->c.layers + 1) * s->c.batch * n_prompt * s->c.d_model * 4;
  float *dev = (float *)nlg_malloc(bytes);
  if (!dev) return NLG_ERR;
  int rc = stack_prefill(s, prompts, n_prompt, dev);
  if (!rc) rc = nlg_download(xs, dev, bytes);  // synchronous: ordered after the prefill
  nlg_free(dev);
  return rc;
}

extern "C" int nlg_stack_step(nlg_stack *s, uint32_t steps, int use_graph) {
  if (!s || !s->started) return nlg_fail("stack step: not started");
  if (s->tiled && stack_tile(s)) return NLG_ERR;
  if ((uint64_t)s->host_pos + steps > s->c.max_seq)
    return nlg_fail("stack step: %u steps from position %u pass max_seq %u", steps, s->host_pos, s->c.max_seq);
  if (use_graph && !s->graph) {
    if (nlg_graph_begin(nullptr)) return NLG_ERR;
    const int rc = stack_enqueue(s);
    void *g = nullptr;
    const int rc2 = nlg_graph_end(nullptr, &g);
    if (rc || rc2) {
      if (g) nlg_graph_destroy(g);
      return NLG_ERR;
    }
    s->graph = g;
  }
  for (uint32_t i = 0; i < steps; i++) {
    if (use_graph ? nlg_graph_launch(s->graph, nullptr) : stack_enqueue(s)) return NLG_ERR;
  }
  NLG_HIP(hipStreamSynchronize(nlg_stream(nullptr)));
  s->host_pos += steps;
  return NLG_OK;
}

extern "C" int nlg_stack_step_trace(nlg_stack *s, float *xs) {
  if (!s || !s->started) return nlg_fail("stack step trace: not started");
  if (!xs) return nlg_fail("stack step trace: null argument");
  if ((uint64_t)s->host_pos + 1 > s->c.max_seq)
    return nlg_fail("stack step trace: position %u is at max_seq %u", s->host_pos, s->c.max_seq);
  if (s->tiled && stack_tile(s)) return NLG_ERR;
  const size_t bytes = (size_t)(s->c.layers + 1) * s->c.batch * s->c.d_model * 4;
  float *dev = (float *)nlg_malloc(bytes);
  if (!dev) return NLG_ERR;
  int rc = stack_enqueue(s, dev);
  if (!rc) rc = nlg_download(xs, dev, bytes);  // synchronous: ordered after the step
  nlg_free(dev);
  if (!rc) s->host_pos += 1;
  return rc;
}

extern "C" int nlg_stack_position(nlg_stack *s, uint32_t *pos) {
  if (!s || !pos) return nlg_fail("stack position: null argument");
  *pos = s->host_pos;
  return NLG_OK;
}

extern "C" int nlg_stack_tokens(nlg_stack *s, int32_t *tokens, int32_t *greedy) {
  if (!s) return nlg_fail("stack tokens: null stack");
  const size_t n = (size_t)s->c.batch * s->c.max_seq * 4;
  if (tokens && nlg_download(tokens, s->hist, n)) return NLG_ERR;
  if (greedy && nlg_download(greedy, s->greedy, n)) return NLG_ERR;
  return NLG_OK;
}

extern "C" int nlg_stack_logits(nlg_stack *s, float *logits) {
  if (!s || !logits) return nlg_fail("stack logits: null argument");
  return nlg_download(logits, s->logits, (size_t)s->c.batch * s->c.vocab * 4);
}

extern "C" int nlg_stack_tensor(nlg_stack *s, const char *name, int layer, void **ptr, size_t *bytes) {
  if (!s || !name || !ptr || !bytes) return nlg_fail("stack tensor: null argument");
  const nlg_stack_config &c = s->c;
  const uint32_t d = c.d_model, f = c.d_ff, qkv = s->nq + 2 * s->nkv;
  const size_t cache = (size_t)c.batch * c.kv_heads * c.max_seq * c.head_dim * 2;
  struct Ent { const char *n; void *p; size_t b; };
  if (layer >= 0) {
    if ((uint32_t)layer >= c.layers) return nlg_fail("stack tensor: layer %d out of range", layer);
    Layer &y = s->L[layer];
    const Ent t[] = {{"wqkv", y.wqkv, (size_t)qkv * (d / 16) * 4}, {"bqkv", y.bqkv, (size_t)qkv * 4},
                     {"wo", y.wo, (size_t)d * (s->nq / 16) * 4},   {"bo", y.bo, 4},
                     {"wgu", y.wgu, (size_t)2 * f * (d / 16) * 4}, {"bgu", y.bgu, (size_t)2 * f * 4},
                     {"wd", y.wd, (size_t)d * (f / 16) * 4},       {"bd", y.bd, 4},
                     {"gattn", y.gattn, (size_t)d * 4},            {"gffn", y.gffn, (size_t)d * 4},
                     {"kc", y.kc, cache},                          {"vc", y.vc, cache}};
    for (const Ent &e : t)
      if (!strcmp(e.n, name)) {
        *ptr = e.p;
        *bytes = e.b;
        if (name[0] == 'w') s->retile = true;  // wqkv, wo, wgu, wd: may be written
        return NLG_OK;
      }
  } else {
    const size_t half = c.head_dim / 2;
    const Ent t[] = {{"wlm", s->wlm, (size_t)c.vocab * (d / 16) * 4}, {"blm", s->blm, 4},
                     {"gfinal", s->gfinal, (size_t)d * 4},           {"emb", s->emb, (size_t)c.vocab * d * 4},
                     {"rope_cos", s->co, c.max_seq * half * 4},      {"rope_sin", s->si, c.max_seq * half * 4},
                     {"x", s->x, (size_t)c.batch * d * 4}};
    for (const Ent &e : t)
      if (!strcmp(e.n, name)) {
        *ptr = e.p;
        *bytes = e.b;
        if (!strcmp(name, "wlm")) s->retile = true;
        return NLG_OK;
      }
  }
  return nlg_fail("stack tensor: no tensor '%s' (layer %d)", name, layer);
}
