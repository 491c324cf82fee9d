/* vksoftmax.c -- row softmax check host on MI355X.
 *
 *   vksoftmax SPV [M N]          (default 64 x 256)
 *
 * As host/vksoftmax.c:36-116: input (i%7)*0.3, one dispatch of (M+63)/64
 * groups, sampled check against double with absolute tolerance 1e-3, and the
 * row-0 sum.  Same output line; exit 1 on a failed sample.
 */
#include <math.h>

#include "nlg_host.h"

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s softmax.spv [M N]\n", argv[0]);
    return 1;
  }
  uint32_t M = (argc >= 4) ? (uint32_t)atoi(argv[2]) : 64, N = (argc >= 4) ? (uint32_t)atoi(argv[3]) : 256;
  size_t sz = (size_t)M * N;
  nlgh_init_or_die("vksoftmax");
  char dev[256];
  nlgh_check(nlg_device_name(dev, sizeof dev), "vksoftmax");
  printf("device = %s\n", dev);
  float *h = malloc(sz * 4 + 4);
  for (size_t i = 0; i < sz; i++) h[i] = (float)((i % 7)) * 0.3f;
  void *A = nlg_malloc(sz * 4), *C = nlg_malloc(sz * 4);
  if (!A || !C) nlgh_check(NLG_ERR, "vksoftmax");
  nlgh_check(nlg_upload(A, h, sz * 4), "vksoftmax");
  nlg_buffer bufs[2] = {{A, (uint32_t)sz}, {C, (uint32_t)sz}};
  uint32_t pc[2] = {M, N};
  nlgh_check(nlg_dispatch("softmax", bufs, 2, pc, 2, (M + 63) / 64, NULL), "vksoftmax");
  nlgh_check(nlg_download(h, C, sz * 4), "vksoftmax");
  int bad = 0;
  double maxerr = 0;
  for (uint32_t r = 0; r < M && bad < 5; r += (M / 9 > 0 ? M / 9 : 1)) {
    double mx = -1e30;
    for (uint32_t j = 0; j < N; j++) {
      double v = (double)(((size_t)r * N + j) % 7) * 0.3;
      if (v > mx) mx = v;
    }
    double s = 0;
    for (uint32_t j = 0; j < N; j++) s += exp((double)(((size_t)r * N + j) % 7) * 0.3 - mx);
    for (uint32_t j = 0; j < N; j += (N / 9 > 0 ? N / 9 : 1)) {
      double ref = exp((double)(((size_t)r * N + j) % 7) * 0.3 - mx) / s;
      double got = h[(size_t)r * N + j];
      double err = fabs(got - ref);
      if (err > maxerr) maxerr = err;
      if (err > 1e-3) {
        if (bad < 5) fprintf(stderr, "C[%u,%u]=%g ref=%g\n", r, j, got, ref);
        bad++;
      }
    }
  }
  double rs = 0;
  for (uint32_t j = 0; j < N; j++) rs += h[j];
  printf("softmax %ux%u  row0_sum=%.5f  max_abs_err=%.2e  %s\n", M, N, rs, maxerr, bad ? "FAIL" : "PASS");
  nlg_free(A);
  nlg_free(C);
  nlg_shutdown();
  return bad ? 1 : 0;
}
