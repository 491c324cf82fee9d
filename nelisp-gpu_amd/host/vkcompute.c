/* vkcompute.c -- vadd smoke host on MI355X.
 *
 *   vkcompute SPV [N]            (default 1024)
 *
 * As host/vkcompute.c:70-235: a = i, b = 2i, c = a + b checked exactly
 * against 3i.  Device selection follows NELISP_GPU_DEVICE (:15-16).  Same
 * output lines; exit 1 on a mismatch, 2 on device errors.
 */
#include "nlg_host.h"

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s shader.spv [N]\n", argv[0]);
    return 1;
  }
  uint32_t N = (argc >= 3) ? (uint32_t)atoi(argv[2]) : 1024;
  size_t bytes = (size_t)N * sizeof(float);
  nlgh_init_or_die("vkcompute");
  char dev[256];
  nlgh_check(nlg_device_name(dev, sizeof dev), "vkcompute");
  const char *e = getenv("NELISP_GPU_DEVICE");
  printf("device[%d] = %s (type %d)\n", e ? atoi(e) : 0, dev, 2 /* discrete */);
  float *ha = malloc(bytes + 4), *hb = malloc(bytes + 4), *hc = malloc(bytes + 4);
  for (uint32_t i = 0; i < N; i++) {
    ha[i] = (float)i;
    hb[i] = (float)(2 * i);
  }
  void *a = nlg_malloc(bytes), *b = nlg_malloc(bytes), *c = nlg_malloc(bytes);
  if (!a || !b || !c) nlgh_check(NLG_ERR, "vkcompute");
  nlgh_check(nlg_upload(a, ha, bytes), "vkcompute");
  nlgh_check(nlg_upload(b, hb, bytes), "vkcompute");
  nlg_buffer bufs[3] = {{a, N}, {b, N}, {c, N}};
  nlgh_check(nlg_dispatch("vadd", bufs, 3, &N, 1, (N + 63) / 64, NULL), "vkcompute");
  nlgh_check(nlg_download(hc, c, bytes), "vkcompute");
  int bad = 0;
  for (uint32_t i = 0; i < N; i++) {
    float want = (float)i + (float)(2 * i);
    if (hc[i] != want) {
      if (bad < 5) fprintf(stderr, "mismatch i=%u got=%g want=%g\n", i, hc[i], want);
      bad++;
    }
  }
  printf("N=%u  c[0]=%g c[1]=%g c[last]=%g  %s\n", N, N ? hc[0] : 0.0f, (N > 1 ? hc[1] : 0.0f),
         N ? hc[N - 1] : 0.0f, bad ? "FAIL" : "PASS");
  nlg_free(a);
  nlg_free(b);
  nlg_free(c);
  nlg_shutdown();
  return bad ? 1 : 0;
}
