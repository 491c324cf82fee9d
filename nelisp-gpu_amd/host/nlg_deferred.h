/* nlg_deferred.h -- device pointers whose free must wait.
 *
 * The server frees a resident buffer when the client asks (OP_FREE), but a
 * compiled batch may still bind it (the reference leaves that binding
 * dangling, host/vkserver.c:412-418 with :536); such pointers are parked here
 * and freed once no compiled batch binds them.  The table grows as needed and
 * reuses the slots of pointers already freed, so a pointer that is still
 * bound is never freed, however many are parked.
 */
#ifndef NLG_DEFERRED_H
#define NLG_DEFERRED_H

#include <stdlib.h>

typedef struct {
  void **p;      /* parked pointers; NULL marks a free slot */
  size_t n, cap; /* slots in use (high-water mark), allocated */
} nlg_deferred;

/* Park p.  Returns 0, or -1 if the table could not grow (p is then not
 * parked and the caller must keep it). */
static inline int nlg_deferred_add(nlg_deferred *d, void *p) {
  for (size_t i = 0; i < d->n; i++)
    if (!d->p[i]) {
      d->p[i] = p;
      return 0;
    }
  if (d->n == d->cap) {
    size_t cap = d->cap ? 2 * d->cap : 64;
    void **q = (void **)realloc(d->p, cap * sizeof *q);
    if (!q) return -1;
    d->p = q;
    d->cap = cap;
  }
  d->p[d->n++] = p;
  return 0;
}

/* Free, with free_fn, every parked pointer bound_fn says nothing binds any
 * more; returns how many were freed. */
static inline size_t nlg_deferred_sweep(nlg_deferred *d, int (*bound_fn)(const void *), void (*free_fn)(void *)) {
  size_t freed = 0;
  for (size_t i = 0; i < d->n; i++)
    if (d->p[i] && !bound_fn(d->p[i])) {
      free_fn(d->p[i]);
      d->p[i] = NULL;
      freed++;
    }
  while (d->n && !d->p[d->n - 1]) d->n--;
  return freed;
}

/* Number of pointers parked now. */
static inline size_t nlg_deferred_count(const nlg_deferred *d) {
  size_t c = 0;
  for (size_t i = 0; i < d->n; i++) c += d->p[i] != NULL;
  return c;
}

#endif /* NLG_DEFERRED_H */
