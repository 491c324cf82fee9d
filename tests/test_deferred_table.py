"""The server's table of deferred frees (nelisp-gpu_amd/host/nlg_deferred.h),
compiled on the CPU with a fake device: a pointer a compiled batch still
binds is never freed, slots of freed pointers are reused, and the table
grows past any fixed size (the reference frees such a resident at once and
leaves the batch's binding dangling, host/vkserver.c:412-418, :536)."""
import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = r'''
#include <stdio.h>
#include "nlg_deferred.h"
static char bound[100000], freed[100000];
static char base[100000];
static int is_bound(const void *p) { return bound[(const char *)p - base]; }
static void do_free(void *p) {
  long i = (char *)p - base;
  if (bound[i]) { printf("FREED A BOUND POINTER %ld\n", i); exit(1); }
  if (freed[i]) { printf("DOUBLE FREE %ld\n", i); exit(1); }
  freed[i] = 1;
}
int main(void) {
  nlg_deferred d = {0};
  /* park 20000 bound pointers (more than the 4096 resident slots) */
  for (int i = 0; i < 20000; i++) { bound[i] = 1; if (nlg_deferred_add(&d, base + i)) return 2; }
  if (nlg_deferred_count(&d) != 20000) return 3;
  /* a batch goes away: the even ones are unbound, the odd ones stay */
  for (int i = 0; i < 20000; i += 2) bound[i] = 0;
  if (nlg_deferred_sweep(&d, is_bound, do_free) != 10000) return 4;
  if (nlg_deferred_count(&d) != 10000) return 5;
  /* parking more reuses the freed slots before growing */
  size_t cap = d.cap, n = d.n;
  for (int i = 20000; i < 25000; i++) { bound[i] = 1; nlg_deferred_add(&d, base + i); }
  if (d.cap != cap || d.n != n) return 6;
  /* unbinding the middle leaves the ends; a sweep with nothing unbound frees nothing */
  if (nlg_deferred_sweep(&d, is_bound, do_free) != 0) return 7;
  for (int i = 0; i < 25000; i++) bound[i] = 0;
  if (nlg_deferred_sweep(&d, is_bound, do_free) != 15000 || d.n != 0) return 8;
  for (int i = 0; i < 25000; i++) if (!freed[i]) { printf("leaked %d\n", i); return 9; }
  printf("ok\n");
  return 0;
}
'''


def test_deferred_frees_never_free_a_bound_pointer():
    with tempfile.TemporaryDirectory() as t:
        src, exe = os.path.join(t, "d.c"), os.path.join(t, "d")
        open(src, "w").write(PROGRAM)
        subprocess.run(["gcc", "-O1", "-Wall", "-I", os.path.join(ROOT, "nelisp-gpu_amd", "host"), src, "-o", exe],
                       check=True)
        p = subprocess.run([exe], capture_output=True, text=True)
        assert p.returncode == 0 and p.stdout.strip() == "ok", (p.returncode, p.stdout)
