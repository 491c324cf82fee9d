/* vkrun.c -- one-shot kernel dispatcher on MI355X.
 *
 *   vkrun SPV IN_FILE OUT_FILE LOCAL GROUPS PUSH_CSV SIZES_CSV
 *
 * Same arguments, files and exit codes as the reference (host/vkrun.c:11-13):
 * IN_FILE holds every buffer's floats in binding order (a short file is
 * zero-padded, :41-45), the kernel runs once as GROUPS workgroups, and
 * OUT_FILE receives ALL buffers back in binding order (:125-129).  LOCAL is
 * accepted and ignored, as in the reference.  PUSH_CSV "-" means none.
 * SPV names the kernel: "name:<kernel>", or a path whose basename is the
 * kernel name (kernels/matmul.spv), or any path with NLG_KERNEL=<kernel> set.
 * Exit 0 on success, 1 for usage, 2 for I/O, device or dispatch errors.
 */
#include "nlg_host.h"

int main(int argc, char **argv) {
  if (argc < 8) {
    fprintf(stderr, "usage: %s SPV IN OUT LOCAL GROUPS PUSH SIZES\n", argv[0]);
    return 1;
  }
  const char *inp = argv[2], *outp = argv[3];
  uint32_t groups = (uint32_t)strtoul(argv[5], NULL, 10);
  uint32_t push[16], sizes[16];
  int npush = nlgh_parse_csv(argv[6], push, 16);
  int nbuf = nlgh_parse_csv(argv[7], sizes, 16);
  if (nbuf < 1) {
    fprintf(stderr, "need >=1 buffer\n");
    return 1;
  }
  size_t total = 0;
  for (int i = 0; i < nbuf; i++) total += sizes[i];
  float *host = calloc(total ? total : 1, 4);
  {
    FILE *f = fopen(inp, "rb");
    if (!f) {
      fprintf(stderr, "open %s\n", inp);
      return 2;
    }
    size_t got = fread(host, 4, total, f);
    fclose(f);
    (void)got; /* calloc already zero-padded a short file */
  }
  char name[256];
  if (!nlgh_kernel_from_arg(argv[1], name, sizeof name)) {
    fprintf(stderr, "vkrun: cannot tell which kernel %s is (use name:<kernel> or NLG_KERNEL)\n", argv[1]);
    return 2;
  }
  nlgh_init_or_die("vkrun");
  nlg_buffer bufs[16];
  size_t off = 0;
  for (int i = 0; i < nbuf; i++) {
    bufs[i].ptr = nlg_malloc((size_t)sizes[i] * 4);
    bufs[i].nfloats = sizes[i];
    if (!bufs[i].ptr) nlgh_check(NLG_ERR, "vkrun");
    nlgh_check(nlg_upload(bufs[i].ptr, host + off, (size_t)sizes[i] * 4), "vkrun");
    off += sizes[i];
  }
  nlgh_check(nlg_dispatch(name, bufs, (uint32_t)nbuf, push, (uint32_t)npush, groups, NULL), "vkrun");
  nlgh_check(nlg_stream_sync(NULL), "vkrun");
  off = 0;
  for (int i = 0; i < nbuf; i++) {
    nlgh_check(nlg_download(host + off, bufs[i].ptr, (size_t)sizes[i] * 4), "vkrun");
    off += sizes[i];
  }
  FILE *of = fopen(outp, "wb");
  if (!of) {
    fprintf(stderr, "open %s\n", outp);
    return 2;
  }
  fwrite(host, 4, total, of);
  fclose(of);
  /* explicit teardown, as the reference learned to do (vkrun.c:131-148) */
  for (int i = 0; i < nbuf; i++) nlg_free(bufs[i].ptr);
  nlg_shutdown();
  free(host);
  return 0;
}
