/* nlg_host.h -- helpers shared by the CLI hosts (header-only, C11). */
#ifndef NLG_HOST_H
#define NLG_HOST_H

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../../include/nlgpu.h"

/* Bring the GPU up with the reference's device policy (NELISP_GPU_DEVICE,
 * vkcompute.c:15-16); on failure print and exit 2 as VK_CHECK does. */
static inline void nlgh_init_or_die(const char *who) {
  if (nlg_init(-1) != NLG_OK) {
    fprintf(stderr, "%s: %s\n", who, nlg_last_error());
    exit(2);
  }
}

static inline void nlgh_check(int rc, const char *who) {
  if (rc != NLG_OK) {
    fprintf(stderr, "%s: %s\n", who, nlg_last_error());
    exit(2);
  }
}

/* "1,2,3" -> up to max values; "-" or NULL -> 0 values (vkrun.c:23-26). */
static inline int nlgh_parse_csv(const char *s, uint32_t *out, int max) {
  if (!s || !strcmp(s, "-")) return 0;
  int n = 0;
  char *tmp = strdup(s), *save = NULL;
  for (char *t = strtok_r(tmp, ",", &save); t && n < max; t = strtok_r(NULL, ",", &save))
    out[n++] = (uint32_t)strtoul(t, NULL, 10);
  free(tmp);
  return n;
}

/* Which kernel a .spv argument names.  The reference loads whatever SPIR-V
 * module the path holds; here kernels are compiled in, so the name comes
 * from the argument: "name:<kernel>" literally, else the file's basename
 * without its extension (kernels/matmul.spv -> matmul, Makefile:62), else
 * the environment variable NLG_KERNEL for callers that pass a random
 * temporary path (lisp/nelisp-gpu-run.el:93). */
static inline int nlgh_kernel_from_arg(const char *arg, char *name, size_t len) {
  if (!strncmp(arg, "name:", 5)) {
    snprintf(name, len, "%s", arg + 5);
    return nlg_kernel_lookup(name) >= 0;
  }
  const char *b = strrchr(arg, '/');
  b = b ? b + 1 : arg;
  snprintf(name, len, "%s", b);
  char *dot = strrchr(name, '.');
  if (dot) *dot = 0;
  if (nlg_kernel_lookup(name) >= 0) return 1;
  const char *e = getenv("NLG_KERNEL");
  if (e) {
    snprintf(name, len, "%s", e);
    return nlg_kernel_lookup(name) >= 0;
  }
  return 0;
}

static inline double nlgh_now(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return t.tv_sec + t.tv_nsec * 1e-9;
}

#endif
