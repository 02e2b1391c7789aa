/* CPU restatement of quotebound's gated delta rule. Test infrastructure only: see gdn_ref.h. */
#include "gdn_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int gdn_ref_num_seqs(const gdn_ref_shape* sh) { return sh->cu_seqlens ? sh->n_seqs : sh->B; }

long gdn_ref_num_chunks(const gdn_ref_shape* sh) {
  if (!sh->cu_seqlens) return (long)sh->B * ((sh->T + sh->chunk - 1) / sh->chunk);
  long slots = 0;
  for (int n = 0; n < sh->n_seqs; ++n) {
    const int l = sh->cu_seqlens[n + 1] - sh->cu_seqlens[n];
    slots += (l + sh->chunk - 1) / sh->chunk;
  }
  return slots;
}

int gdn_ref_check(const gdn_ref_shape* sh) {
  if (!sh || sh->B < 1 || sh->T < 0 || sh->Hk < 1 || sh->Hv < 1 || sh->Dk < 1 || sh->Dv < 1 || sh->chunk < 1)
    return -1;
  if (sh->Hv % sh->Hk) return -1;
  if (sh->cu_seqlens) {
    if (sh->B != 1 || sh->n_seqs < 1 || sh->cu_seqlens[0] != 0 || sh->cu_seqlens[sh->n_seqs] != sh->T) return -1;
    for (int n = 0; n < sh->n_seqs; ++n)
      if (sh->cu_seqlens[n + 1] < sh->cu_seqlens[n]) return -1;
  }
  return 0;
}

int gdn_ref_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void gdn_ref_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

#define REAL float
#define SUFFIX _f32
#define EXP expf
#include "gdn_ref_impl.h"
#undef REAL
#undef SUFFIX
#undef EXP

#define REAL double
#define SUFFIX _f64
#define EXP exp
#include "gdn_ref_impl.h"
#undef REAL
#undef SUFFIX
#undef EXP
