/* vkmatmul.c -- f32 matmul check + timing host on MI355X.
 *
 *   vkmatmul SPV [M K N [naive|tiled|reg [iters]]]
 *
 * As host/vkmatmul.c:51-186: A = i%4, B = i%3 (exact in f32), `iters`
 * (default 20) dispatches back to back after one warm-up pass, then a
 * sampled exact check against a double-precision sum.  The variant picks
 * the kernel name (matmul / matmul-tiled / matmul-reg) and its group count
 * (:147-150); SPV may also name it by basename.  Output line format is the
 * reference's (:182-183); exit 1 on a wrong entry.
 */
#include "nlg_host.h"

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s matmul.spv [M K N]\n", argv[0]);
    return 1;
  }
  uint32_t M = (argc >= 5) ? (uint32_t)atoi(argv[2]) : 128;
  uint32_t K = (argc >= 5) ? (uint32_t)atoi(argv[3]) : 128;
  uint32_t N = (argc >= 5) ? (uint32_t)atoi(argv[4]) : 128;
  size_t na = (size_t)M * K, nb = (size_t)K * N, nc = (size_t)M * N;
  nlgh_init_or_die("vkmatmul");
  char dev[256];
  nlgh_check(nlg_device_name(dev, sizeof dev), "vkmatmul");
  printf("device = %s\n", dev);
  float *ha = malloc(na * 4 + 4), *hb = malloc(nb * 4 + 4), *hc = malloc(nc * 4 + 4);
  for (size_t i = 0; i < na; i++) ha[i] = (float)(i % 4);
  for (size_t i = 0; i < nb; i++) hb[i] = (float)(i % 3);
  void *A = nlg_malloc(na * 4), *B = nlg_malloc(nb * 4), *C = nlg_malloc(nc * 4);
  if (!A || !B || !C) nlgh_check(NLG_ERR, "vkmatmul");
  nlgh_check(nlg_upload(A, ha, na * 4), "vkmatmul");
  nlgh_check(nlg_upload(B, hb, nb * 4), "vkmatmul");
  const char *kname = "matmul";
  uint32_t groups;
  if (argc >= 6 && !strcmp(argv[5], "tiled")) {
    kname = "matmul-tiled";
    groups = ((M + 15) / 16) * ((N + 15) / 16);
  } else if (argc >= 6 && !strcmp(argv[5], "reg")) {
    kname = "matmul-reg";
    groups = ((((M + 3) / 4) * ((N + 3) / 4)) + 63) / 64;
  } else {
    char nm[256];
    if (argc < 6 && nlgh_kernel_from_arg(argv[1], nm, sizeof nm) && !strcmp(nm, "matmul-tiled")) {
      kname = "matmul-tiled";
      groups = ((M + 15) / 16) * ((N + 15) / 16);
    } else {
      groups = ((uint32_t)nc + 63) / 64;
    }
  }
  uint32_t iters = (argc >= 7) ? (uint32_t)atoi(argv[6]) : 20;
  if (!iters) iters = 1;
  nlg_buffer bufs[3] = {{A, (uint32_t)na}, {B, (uint32_t)nb}, {C, (uint32_t)nc}};
  uint32_t pc[3] = {M, K, N};
  /* warm-up pass, then the timed pass (vkmatmul.c:163-169) */
  for (uint32_t it = 0; it < iters; it++)
    nlgh_check(nlg_dispatch(kname, bufs, 3, pc, 3, groups, NULL), "vkmatmul");
  nlgh_check(nlg_stream_sync(NULL), "vkmatmul");
  void *e0 = nlg_event_create(), *e1 = nlg_event_create();
  nlg_event_record(e0, NULL);
  for (uint32_t it = 0; it < iters; it++)
    nlgh_check(nlg_dispatch(kname, bufs, 3, pc, 3, groups, NULL), "vkmatmul");
  nlg_event_record(e1, NULL);
  float ms = 0;
  nlgh_check(nlg_event_elapsed_ms(e0, e1, &ms), "vkmatmul");
  double dt = (ms * 1e-3) / (double)iters;
  nlgh_check(nlg_download(hc, C, nc * 4), "vkmatmul");
  int bad = 0;
  size_t checks = 0;
  for (uint32_t r = 0; r < M && bad < 5; r += (M / 7 > 0 ? M / 7 : 1))
    for (uint32_t c = 0; c < N && bad < 5; c += (N / 7 > 0 ? N / 7 : 1)) {
      double acc = 0;
      for (uint32_t k = 0; k < K; k++)
        acc += (double)(((size_t)r * K + k) % 4) * (double)(((size_t)k * N + c) % 3);
      float got = hc[(size_t)r * N + c];
      if ((double)got != acc) {
        if (bad < 5) fprintf(stderr, "C[%u,%u]=%g want=%g\n", r, c, got, acc);
        bad++;
      }
      checks++;
    }
  double flop = 2.0 * (double)M * N * K;
  printf("matmul %ux%u x %ux%u  gpu=%.4fs  %.1f GFLOP/s  checks=%zu  %s\n", M, K, K, N, dt,
         flop / dt / 1e9, checks, bad ? "FAIL" : "PASS");
  nlg_free(A);
  nlg_free(B);
  nlg_free(C);
  nlg_shutdown();
  return bad ? 1 : 0;
}
