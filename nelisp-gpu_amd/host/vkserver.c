/* vkserver.c -- persistent GPU compute server on MI355X, speaking the
 * reference's binary stdin/stdout protocol byte for byte, so
 * lisp/nelisp-gpu-server.el drives it unchanged.
 *
 *   run:   vkserver KERNEL_DIR
 *
 * KERNEL_DIR is accepted and ignored: the client still compiles .spv files
 * into it (lisp/nelisp-gpu-server.el:60-88), but every kernel name resolves
 * to a compiled-in gfx950 kernel through libnlgpu's name table.
 *
 * Protocol (host/vkserver.c:11-38, :420-432, :508-510, :589-590; all
 * integers u32 little-endian, floats raw f32 bytes, never converted):
 *   0 RUN            name, per-buffer (size, kind[, handle]), push, groups,
 *                    inline f32 for kinds 0 and 3     -> status, f32 of kinds 2,3
 *   1 UPLOAD         n, f32[n]                        -> status, handle
 *   2 FREE           handle                           -> status (always 0)
 *   3 BATCH          slots (kind, size[, handle]), dispatches, inline f32
 *                    for kind-0 slots                 -> status, f32 of kind-3 slots
 *   4 COMPILE        as BATCH                         -> status, handle
 *   5 RUN_COMPILED   handle                           -> status, f32 of kind-3 slots
 *   6 FREE_COMPILED  handle                           -> status (always 0)
 *   7 WRITE_RESIDENT handle, n, f32[n]                -> status
 *   8 UPLOAD_FILE    pathlen, path, off_lo, off_hi, n -> status, handle
 *
 * Where this server differs from the reference, it is to keep the stream in
 * sync or the GPU safe, never in the bytes of a successful exchange:
 *   - a RUN or BATCH that fails (unknown kernel, short buffer, bad resident
 *     handle) consumes its whole request and replies status 1 followed by
 *     zeros for every float the client expects, instead of exit(2);
 *   - COMPILE with a full table consumes the inline floats before replying
 *     (the reference replies first and then reads them as opcodes);
 *   - WRITE_RESIDENT past a buffer's end replies 1;
 *   - FREE of a resident still bound by a compiled batch defers the device
 *     free until that batch is freed, so a replay never touches freed memory.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nlg_deferred.h"
#include "nlg_host.h"

#define OP_RUN 0
#define OP_UPLOAD 1
#define OP_FREE 2
#define OP_BATCH 3
#define OP_COMPILE 4
#define OP_RUN_COMPILED 5
#define OP_FREE_COMPILED 6
#define OP_WRITE_RESIDENT 7
#define OP_UPLOAD_FILE 8

#define MAXRES 4096  /* vkserver.c:84 */
#define MAXCOMP 16   /* :93 */
#define MAXSLOT 8192 /* :435 */
#define MAXDISP 8192 /* :436 */

/* ------------------------------------------------------------------ I/O */

static int rd_u32(uint32_t *v) { return fread(v, 4, 1, stdin) == 1; }
static int rd_bytes(void *p, size_t n) { return n == 0 || fread(p, 1, n, stdin) == n; }
static void wr_u32(uint32_t v) { fwrite(&v, 4, 1, stdout); }
static void wr_zero_floats(uint64_t n) {
  static const uint32_t z[1024];
  while (n) {
    size_t k = n > 1024 ? 1024 : (size_t)n;
    fwrite(z, 4, k, stdout);
    n -= k;
  }
}
static void die(const char *msg) {
  fprintf(stderr, "vkserver: %s\n", msg);
  exit(2);
}
/* EOF in the middle of a request ends the server quietly (vkserver.c:275-283). */
static void need_u32(uint32_t *v) {
  if (!rd_u32(v)) exit(0);
}

static void *host_buf(size_t bytes) {
  static void *p = NULL;
  static size_t cap = 0;
  if (bytes > cap) {
    free(p);
    cap = bytes < (1u << 20) ? (1u << 20) : bytes;
    p = malloc(cap);
    if (!p) die("host allocation failed");
  }
  return p;
}

/* Read n floats from stdin straight into device memory (chunked through a
 * host buffer).  Returns 0, or exits on EOF like the reference. */
static void read_into_device(void *dev, uint64_t nfloats) {
  const uint64_t chunk = 1u << 22; /* 16 MiB */
  uint64_t done = 0;
  while (done < nfloats) {
    uint64_t n = nfloats - done;
    if (n > chunk) n = chunk;
    void *h = host_buf((size_t)n * 4);
    if (!rd_bytes(h, (size_t)n * 4)) exit(0);
    if (dev && nlg_upload((char *)dev + done * 4, h, (size_t)n * 4) != NLG_OK) die(nlg_last_error());
    done += n;
  }
}
static void write_from_device(const void *dev, uint64_t nfloats) {
  const uint64_t chunk = 1u << 22;
  uint64_t done = 0;
  while (done < nfloats) {
    uint64_t n = nfloats - done;
    if (n > chunk) n = chunk;
    void *h = host_buf((size_t)n * 4);
    if (nlg_download(h, (const char *)dev + done * 4, (size_t)n * 4) != NLG_OK) die(nlg_last_error());
    fwrite(h, 4, (size_t)n, stdout);
    done += n;
  }
}

/* ------------------------------------------------------ transient pool */

typedef struct {
  void *p;
  size_t cap;
} PBuf;
#define POOLMAX 512
static PBuf g_pool[POOLMAX];
static int g_npool = 0;

static size_t round_cap(size_t bytes) {
  size_t c = 256;
  while (c < bytes) c <<= 1;
  return c;
}
/* A zero-filled device buffer of at least `bytes`. */
static void *pool_get(size_t bytes, size_t *cap_out) {
  size_t cap = round_cap(bytes ? bytes : 4);
  for (int i = 0; i < g_npool; i++)
    if (g_pool[i].cap == cap) {
      void *p = g_pool[i].p;
      g_pool[i] = g_pool[--g_npool];
      if (nlg_zero(p, cap, NULL) != NLG_OK) die(nlg_last_error());
      *cap_out = cap;
      return p;
    }
  void *p = nlg_malloc(cap);
  if (!p) {
    /* release the cache and retry once before giving up */
    for (int i = 0; i < g_npool; i++) nlg_free(g_pool[i].p);
    g_npool = 0;
    p = nlg_malloc(cap);
  }
  *cap_out = cap;
  return p;
}
static void pool_put(void *p, size_t cap) {
  if (!p) return;
  if (g_npool < POOLMAX && cap <= (256u << 20)) {
    g_pool[g_npool].p = p;
    g_pool[g_npool].cap = cap;
    g_npool++;
  } else {
    nlg_free(p);
  }
}

/* ------------------------------------------------------------ residents */

typedef struct {
  void *p;
  uint32_t size;
  int used;
} Res;
static Res g_res[MAXRES];
static int g_nres = 0;

/* first free slot, else a new one (vkserver.c:341-345); -1 when full */
static int res_slot(void) {
  for (int i = 0; i < g_nres; i++)
    if (!g_res[i].used) return i;
  if (g_nres >= MAXRES) return -1;
  return g_nres++;
}
static int res_valid(uint32_t h) { return h < (uint32_t)g_nres && g_res[h].used; }

/* pointers freed by the client while a compiled batch still binds them */
static nlg_deferred g_deferred;

/* -------------------------------------------------------------- batches */

typedef struct {
  char name[64];
  uint32_t nbuf, slot[16], npush, push[16], groups;
} Disp;

typedef struct {
  uint32_t nslot, ndisp;
  uint32_t *kind, *size, *handle;
  Disp *disp;
} Batch;

static void batch_free(Batch *b) {
  free(b->kind);
  free(b->size);
  free(b->handle);
  free(b->disp);
  memset(b, 0, sizeof *b);
}

/* Parse the BATCH/COMPILE body up to (not including) the inline floats. */
static void batch_parse(Batch *b) {
  memset(b, 0, sizeof *b);
  need_u32(&b->nslot);
  if (b->nslot > MAXSLOT) {
    fprintf(stderr, "vkserver: nslot %u > %d\n", b->nslot, MAXSLOT);
    exit(2);
  }
  b->kind = calloc(b->nslot + 1, 4);
  b->size = calloc(b->nslot + 1, 4);
  b->handle = calloc(b->nslot + 1, 4);
  for (uint32_t i = 0; i < b->nslot; i++) {
    need_u32(&b->kind[i]);
    need_u32(&b->size[i]);
    if (b->kind[i] == 1) need_u32(&b->handle[i]);
  }
  need_u32(&b->ndisp);
  if (b->ndisp > MAXDISP) {
    fprintf(stderr, "vkserver: ndisp %u > %d\n", b->ndisp, MAXDISP);
    exit(2);
  }
  b->disp = calloc(b->ndisp + 1, sizeof(Disp));
  for (uint32_t d = 0; d < b->ndisp; d++) {
    Disp *D = &b->disp[d];
    uint32_t nl;
    if (!rd_u32(&nl) || nl >= 64) exit(2); /* vkserver.c:447 */
    if (!rd_bytes(D->name, nl)) exit(0);
    need_u32(&D->nbuf);
    if (D->nbuf > 16) die("dispatch binds more than 16 buffers");
    for (uint32_t i = 0; i < D->nbuf; i++) need_u32(&D->slot[i]);
    need_u32(&D->npush);
    if (D->npush > 16) die("dispatch pushes more than 16 constants");
    for (uint32_t i = 0; i < D->npush; i++) need_u32(&D->push[i]);
    need_u32(&D->groups);
  }
}

/* Run the dispatches over slot buffers; 0 on success. */
static int batch_dispatch(const Batch *b, void **ptr, const uint32_t *nfl) {
  for (uint32_t d = 0; d < b->ndisp; d++) {
    const Disp *D = &b->disp[d];
    nlg_buffer bufs[16];
    for (uint32_t i = 0; i < D->nbuf; i++) {
      uint32_t s = D->slot[i];
      if (s >= b->nslot) {
        fprintf(stderr, "vkserver: %s binds slot %u of %u\n", D->name, s, b->nslot);
        return 1;
      }
      bufs[i].ptr = ptr[s];
      bufs[i].nfloats = nfl[s];
    }
    if (nlg_dispatch(D->name, bufs, D->nbuf, D->push, D->npush, D->groups, NULL) != NLG_OK) {
      fprintf(stderr, "vkserver: %s\n", nlg_last_error());
      return 1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------- compiled */

typedef struct {
  int used;
  Batch b;
  void **ptr;
  uint32_t *nfl;
  size_t *cap; /* nonzero for buffers this batch owns */
  void *graph;
} Comp;
static Comp g_comp[MAXCOMP];

static void free_device(void *p) { nlg_free(p); }

static int comp_binds(const void *p) {
  for (int c = 0; c < MAXCOMP; c++)
    if (g_comp[c].used)
      for (uint32_t i = 0; i < g_comp[c].b.nslot; i++)
        if (!g_comp[c].cap[i] && g_comp[c].ptr[i] == p) return 1;
  return 0;
}

static void comp_release(Comp *C) {
  if (C->graph) nlg_graph_destroy(C->graph);
  for (uint32_t i = 0; i < C->b.nslot; i++)
    if (C->cap[i]) nlg_free(C->ptr[i]);
  free(C->ptr);
  free(C->nfl);
  free(C->cap);
  batch_free(&C->b);
  memset(C, 0, sizeof *C);
  /* deferred frees no batch binds any more */
  nlg_deferred_sweep(&g_deferred, comp_binds, free_device);
}

/* Zero this batch's tmp/out slots then run its dispatches. */
static int comp_record(Comp *C) {
  for (uint32_t i = 0; i < C->b.nslot; i++)
    if (C->cap[i] && C->b.kind[i] != 0 && nlg_zero(C->ptr[i], C->cap[i], NULL) != NLG_OK) return 1;
  return batch_dispatch(&C->b, C->ptr, C->nfl);
}

/* -------------------------------------------------------------- handlers */

static void handle_run(void) {
  uint32_t name_len;
  need_u32(&name_len);
  char name[64] = {0};
  if (name_len >= 64) {
    fprintf(stderr, "name too long\n");
    exit(2);
  }
  if (!rd_bytes(name, name_len)) exit(0);
  uint32_t nbuf;
  need_u32(&nbuf);
  if (nbuf > 16) die("run binds more than 16 buffers");
  uint32_t size[16], kind[16], handle[16];
  for (uint32_t i = 0; i < nbuf; i++) {
    need_u32(&size[i]);
    need_u32(&kind[i]);
    handle[i] = 0;
    if (kind[i] == 1) need_u32(&handle[i]);
  }
  uint32_t npush, push[16];
  need_u32(&npush);
  if (npush > 16) die("run pushes more than 16 constants");
  for (uint32_t i = 0; i < npush; i++) need_u32(&push[i]);
  uint32_t groups;
  need_u32(&groups);

  int err = 0;
  nlg_buffer bufs[16];
  size_t cap[16] = {0};
  uint64_t outn = 0;
  for (uint32_t i = 0; i < nbuf; i++) {
    bufs[i].ptr = NULL;
    bufs[i].nfloats = size[i];
    if (kind[i] == 1) {
      if (res_valid(handle[i])) {
        bufs[i].ptr = g_res[handle[i]].p;
        bufs[i].nfloats = g_res[handle[i]].size;
      } else {
        fprintf(stderr, "vkserver: bad resident handle %u\n", handle[i]);
        err = 1;
      }
      continue;
    }
    bufs[i].ptr = pool_get((size_t)size[i] * 4, &cap[i]);
    if (!bufs[i].ptr) {
      fprintf(stderr, "vkserver: %s\n", nlg_last_error());
      err = 1;
    }
    if (kind[i] == 0 || kind[i] == 3) read_into_device(bufs[i].ptr, size[i]);
    if (kind[i] == 2 || kind[i] == 3) outn += size[i];
  }
  if (!err && nlg_dispatch(name, bufs, nbuf, push, npush, groups, NULL) != NLG_OK) {
    fprintf(stderr, "vkserver: %s\n", nlg_last_error());
    err = 1;
  }
  if (!err && nlg_stream_sync(NULL) != NLG_OK) die(nlg_last_error());
  wr_u32(err ? 1u : 0u);
  for (uint32_t i = 0; i < nbuf; i++)
    if (kind[i] == 2 || kind[i] == 3) {
      if (err || !bufs[i].ptr) wr_zero_floats(size[i]);
      else write_from_device(bufs[i].ptr, size[i]);
    }
  fflush(stdout);
  (void)outn;
  for (uint32_t i = 0; i < nbuf; i++)
    if (kind[i] != 1) pool_put(bufs[i].ptr, cap[i]);
}

static void handle_upload(void) {
  uint32_t n;
  need_u32(&n);
  int h = res_slot();
  void *p = h >= 0 ? nlg_malloc((size_t)n * 4) : NULL;
  read_into_device(p, n); /* consumes the floats even when there is nowhere to put them */
  if (!p) {
    fprintf(stderr, h < 0 ? "vkserver: resident table full\n" : "vkserver: %s\n", nlg_last_error());
    if (h >= 0 && h == g_nres - 1 && !g_res[h].used) g_nres--;
    wr_u32(1);
    wr_u32(0);
    fflush(stdout);
    return;
  }
  g_res[h].p = p;
  g_res[h].size = n;
  g_res[h].used = 1;
  wr_u32(0);
  wr_u32((uint32_t)h);
  fflush(stdout);
}

static void release_resident(uint32_t h) {
  void *p = g_res[h].p;
  g_res[h].used = 0;
  g_res[h].p = NULL;
  if (!comp_binds(p)) {
    nlg_free(p);
  } else if (nlg_deferred_add(&g_deferred, p)) {
    /* out of host memory: leak the buffer rather than free one a graph binds */
    fprintf(stderr, "vkserver: cannot park a bound resident; it stays allocated\n");
  }
}

static void handle_free(void) {
  uint32_t h;
  need_u32(&h);
  if (res_valid(h)) release_resident(h);
  wr_u32(0); /* 0 even for an invalid handle (vkserver.c:412-418) */
  fflush(stdout);
}

static void handle_write_resident(void) {
  uint32_t h, n;
  need_u32(&h);
  need_u32(&n);
  int ok = res_valid(h) && n <= g_res[h].size;
  read_into_device(ok ? g_res[h].p : NULL, n);
  if (!ok) fprintf(stderr, "vkserver: write bad resident %u\n", h);
  wr_u32(ok ? 0u : 1u);
  fflush(stdout);
}

static void handle_upload_file(void) {
  uint32_t plen, olo, ohi, n;
  need_u32(&plen);
  if (plen == 0 || plen > 4095) {
    fprintf(stderr, "vkserver: bad path length %u\n", plen);
    exit(0); /* as vkserver.c:374 */
  }
  char path[4096];
  if (!rd_bytes(path, plen)) exit(0);
  path[plen] = 0;
  need_u32(&olo);
  need_u32(&ohi);
  need_u32(&n);
  uint64_t off = ((uint64_t)ohi << 32) | olo;
  FILE *f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "vkserver: cannot open %s\n", path);
    wr_u32(1);
    wr_u32(0);
    fflush(stdout);
    return;
  }
  int seek_ok = fseeko(f, (off_t)off, SEEK_SET) == 0;
  fclose(f);
  if (!seek_ok) {
    fprintf(stderr, "vkserver: seek %s\n", path);
    wr_u32(1);
    wr_u32(0);
    fflush(stdout);
    return;
  }
  int h = res_slot();
  if (h < 0) {
    fprintf(stderr, "vkserver: resident table full\n");
    wr_u32(1);
    wr_u32(0);
    fflush(stdout);
    return;
  }
  void *p = nlg_malloc((size_t)n * 4);
  size_t missing = 0;
  int rc = p ? nlg_upload_file(p, path, off, (size_t)n * 4, &missing) : NLG_ERR;
  if (rc != NLG_OK || missing) {
    if (missing) fprintf(stderr, "vkserver: %s short read, %zu floats missing\n", path, missing / 4);
    else fprintf(stderr, "vkserver: %s\n", nlg_last_error());
    nlg_free(p);
    if (h == g_nres - 1) g_nres--;
    wr_u32(1);
    wr_u32(0);
    fflush(stdout);
    return;
  }
  g_res[h].p = p;
  g_res[h].size = n;
  g_res[h].used = 1;
  wr_u32(0);
  wr_u32((uint32_t)h);
  fflush(stdout);
}

/* Allocate a batch's slot buffers; kind-0 data is read from stdin here. */
static int batch_buffers(const Batch *b, void **ptr, uint32_t *nfl, size_t *cap, int persistent) {
  int err = 0;
  for (uint32_t i = 0; i < b->nslot; i++) {
    ptr[i] = NULL;
    cap[i] = 0;
    nfl[i] = b->size[i];
    if (b->kind[i] == 1) {
      if (res_valid(b->handle[i])) {
        ptr[i] = g_res[b->handle[i]].p;
        nfl[i] = g_res[b->handle[i]].size;
      } else {
        fprintf(stderr, "vkserver: bad resident handle %u\n", b->handle[i]);
        err = 1;
      }
      continue;
    }
    if (persistent) {
      cap[i] = (size_t)(b->size[i] ? b->size[i] : 1) * 4;
      ptr[i] = nlg_malloc(cap[i]);
    } else {
      ptr[i] = pool_get((size_t)b->size[i] * 4, &cap[i]);
    }
    if (!ptr[i]) {
      fprintf(stderr, "vkserver: %s\n", nlg_last_error());
      err = 1;
      cap[i] = 0;
    }
  }
  /* inline data for kind-0 slots, in slot order, after the whole body */
  for (uint32_t i = 0; i < b->nslot; i++)
    if (b->kind[i] == 0) read_into_device(ptr[i], b->size[i]);
  return err;
}

static void handle_batch(void) {
  Batch b;
  batch_parse(&b);
  void **ptr = calloc(b.nslot + 1, sizeof(void *));
  uint32_t *nfl = calloc(b.nslot + 1, 4);
  size_t *cap = calloc(b.nslot + 1, sizeof(size_t));
  int err = batch_buffers(&b, ptr, nfl, cap, 0);
  if (!err) err = batch_dispatch(&b, ptr, nfl);
  if (!err && nlg_stream_sync(NULL) != NLG_OK) die(nlg_last_error());
  wr_u32(err ? 1u : 0u);
  for (uint32_t i = 0; i < b.nslot; i++)
    if (b.kind[i] == 3 && b.size[i]) {
      if (err || !ptr[i]) wr_zero_floats(b.size[i]);
      else write_from_device(ptr[i], b.size[i]);
    }
  fflush(stdout);
  for (uint32_t i = 0; i < b.nslot; i++)
    if (b.kind[i] != 1) pool_put(ptr[i], cap[i]);
  free(ptr);
  free(nfl);
  free(cap);
  batch_free(&b);
}

static void handle_compile(void) {
  Batch b;
  batch_parse(&b);
  int c = -1;
  for (int i = 0; i < MAXCOMP; i++)
    if (!g_comp[i].used) {
      c = i;
      break;
    }
  if (c < 0) {
    for (uint32_t i = 0; i < b.nslot; i++)
      if (b.kind[i] == 0) read_into_device(NULL, b.size[i]);
    fprintf(stderr, "vkserver: compiled table full\n");
    batch_free(&b);
    wr_u32(1);
    wr_u32(0);
    fflush(stdout);
    return;
  }
  Comp *C = &g_comp[c];
  memset(C, 0, sizeof *C);
  C->b = b;
  C->ptr = calloc(b.nslot + 1, sizeof(void *));
  C->nfl = calloc(b.nslot + 1, 4);
  C->cap = calloc(b.nslot + 1, sizeof(size_t));
  C->used = 1;
  int err = batch_buffers(&C->b, C->ptr, C->nfl, C->cap, 1);
  if (!err) {
    /* validate + record once as a graph; fall back to eager replay */
    if (nlg_graph_begin(NULL) == NLG_OK) {
      int rerr = comp_record(C);
      void *g = NULL;
      int gerr = nlg_graph_end(NULL, &g);
      if (rerr) {
        if (!gerr) nlg_graph_destroy(g);
        err = 1;
      } else if (!gerr) {
        C->graph = g;
      }
    }
    if (!err && !C->graph) {
      /* dry-run validation happens on the first run; check names now */
      for (uint32_t d = 0; d < C->b.ndisp; d++)
        if (nlg_kernel_lookup(C->b.disp[d].name) < 0) {
          fprintf(stderr, "vkserver: no kernel named '%s'\n", C->b.disp[d].name);
          err = 1;
        }
    }
  }
  if (err) {
    comp_release(C);
    wr_u32(1);
    wr_u32(0);
  } else {
    wr_u32(0);
    wr_u32((uint32_t)c);
  }
  fflush(stdout);
}

static void handle_run_compiled(void) {
  uint32_t h;
  need_u32(&h);
  if (h >= MAXCOMP || !g_comp[h].used) {
    fprintf(stderr, "vkserver: bad compiled %u\n", h);
    wr_u32(1); /* the reference replies the status alone (vkserver.c:593) */
    fflush(stdout);
    return;
  }
  Comp *C = &g_comp[h];
  int err = C->graph ? (nlg_graph_launch(C->graph, NULL) != NLG_OK) : comp_record(C);
  if (!err && nlg_stream_sync(NULL) != NLG_OK) die(nlg_last_error());
  wr_u32(err ? 1u : 0u);
  for (uint32_t i = 0; i < C->b.nslot; i++)
    if (C->b.kind[i] == 3 && C->b.size[i]) {
      if (err) wr_zero_floats(C->b.size[i]);
      else write_from_device(C->ptr[i], C->b.size[i]);
    }
  fflush(stdout);
}

static void handle_free_compiled(void) {
  uint32_t h;
  need_u32(&h);
  if (h < MAXCOMP && g_comp[h].used) comp_release(&g_comp[h]);
  wr_u32(0);
  fflush(stdout);
}

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s KERNEL_DIR\n", argv[0]);
    return 1;
  }
  static char inbuf[1 << 20], outbuf[1 << 20];
  setvbuf(stdin, inbuf, _IOFBF, sizeof inbuf);
  setvbuf(stdout, outbuf, _IOFBF, sizeof outbuf);
  nlgh_init_or_die("vkserver");
  char dev[256];
  if (nlg_device_name(dev, sizeof dev) != NLG_OK) snprintf(dev, sizeof dev, "?");
  fprintf(stderr, "vkserver: device = %s\n", dev);
  fprintf(stderr, "vkserver: ready\n");
  fflush(stderr);
  uint32_t op;
  while (rd_u32(&op)) {
    if (op == OP_RUN) handle_run();
    else if (op == OP_UPLOAD) handle_upload();
    else if (op == OP_FREE) handle_free();
    else if (op == OP_BATCH) handle_batch();
    else if (op == OP_COMPILE) handle_compile();
    else if (op == OP_RUN_COMPILED) handle_run_compiled();
    else if (op == OP_FREE_COMPILED) handle_free_compiled();
    else if (op == OP_WRITE_RESIDENT) handle_write_resident();
    else if (op == OP_UPLOAD_FILE) handle_upload_file();
    else {
      fprintf(stderr, "vkserver: bad opcode %u\n", op);
      return 2;
    }
  }
  nlg_shutdown();
  return 0;
}
