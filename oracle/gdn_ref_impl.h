/*
 * Body of the oracle, instantiated twice by gdn_ref.c: REAL = float (the reference's own fp32 arithmetic) and
 * REAL = double (the precise value the float paths are measured against). Test infrastructure only.
 */
#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SUFFIX)

/* One value head of one sequence: token and state offsets. */
typedef struct {
  long tok0;   /* flattened index of the sequence's first token in [B*T] */
  int len;     /* steps */
  long slot0;  /* first chunk slot of the sequence in ckpt */
  int n;       /* state index */
} FN(seq_t);

static FN(seq_t) FN(seq_of)(const gdn_ref_shape* sh, int n) {
  FN(seq_t) s;
  s.n = n;
  if (sh->cu_seqlens) {
    s.tok0 = sh->cu_seqlens[n];
    s.len = sh->cu_seqlens[n + 1] - sh->cu_seqlens[n];
    long slots = 0;
    for (int m = 0; m < n; ++m) {
      const int l = sh->cu_seqlens[m + 1] - sh->cu_seqlens[m];
      slots += (l + sh->chunk - 1) / sh->chunk;
    }
    s.slot0 = slots;
  } else {
    s.tok0 = (long)n * sh->T;
    s.len = sh->T;
    s.slot0 = (long)n * ((sh->T + sh->chunk - 1) / sh->chunk);
  }
  return s;
}

/* Decay factor of step tok for value head hv: the input itself, or exp of the log-decay. */
static inline REAL FN(decay)(const gdn_ref_shape* sh, const REAL* g, long idx) {
  return sh->g_is_log ? (REAL)EXP(g[idx]) : g[idx];
}

/* Forward: tests/gated_delta_ref.h:110-118, one value head of one sequence, all rows at once (as the plain-ops
 * oracle does): decay, kv_mem = sum(S k), delta = (v - kv_mem) beta, S += k delta, y = sum(S q). */
int FN(gdn_ref_fwd)(const gdn_ref_shape* sh, const REAL* q, const REAL* k, const REAL* v, const REAL* g,
                    const REAL* beta, const REAL* s0, REAL* y, REAL* s_out, REAL* ckpt) {
  if (gdn_ref_check(sh)) return -1;
  const int N = gdn_ref_num_seqs(sh), Hk = sh->Hk, Hv = sh->Hv, Dk = sh->Dk, Dv = sh->Dv, C = sh->chunk;
  const int grp = Hv / Hk;
  const long SS = (long)Dv * Dk;
  int bad = 0;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int n = 0; n < N; ++n) {
    for (int hv = 0; hv < Hv; ++hv) {
      const FN(seq_t) sq = FN(seq_of)(sh, n);
      const int hk = hv / grp;
      REAL* S = (REAL*)malloc(sizeof(REAL) * SS);
      if (!S) {
#pragma omp atomic write
        bad = 1;
        continue;
      }
      const long st0 = ((long)n * Hv + hv) * SS;
      for (long e = 0; e < SS; ++e) S[e] = s0 ? s0[st0 + e] : (REAL)0;
      for (int t = 0; t < sq.len; ++t) {
        if (t % C == 0 && ckpt) {
          const long c0 = ((sq.slot0 + t / C) * Hv + hv) * SS;
          memcpy(ckpt + c0, S, sizeof(REAL) * SS);
        }
        const long tok = sq.tok0 + t;
        const REAL* kt = k + (tok * Hk + hk) * Dk;
        const REAL* qt = q + (tok * Hk + hk) * Dk;
        const REAL gt = FN(decay)(sh, g, tok * Hv + hv), bt = beta[tok * Hv + hv];
        for (int r = 0; r < Dv; ++r) {
          REAL* s = S + (long)r * Dk;
          REAL u = 0;
          for (int i = 0; i < Dk; ++i) {
            s[i] = s[i] * gt;
            u += s[i] * kt[i];
          }
          const REAL d = (v[(tok * Hv + hv) * Dv + r] - u) * bt;
          REAL o = 0;
          for (int i = 0; i < Dk; ++i) {
            s[i] = s[i] + kt[i] * d;
            o += s[i] * qt[i];
          }
          y[(tok * Hv + hv) * Dv + r] = o;
        }
      }
      if (s_out) memcpy(s_out + st0, S, sizeof(REAL) * SS);
      free(S);
    }
  }
  return bad ? -1 : 0;
}

/* Backward: src/delta_grad.cpp:97-141 for each state row, chunk by chunk in reverse from the checkpoints, each
 * chunk's states recomputed from its start (:54-95). Parallel over (sequence, key head): the value heads of a key
 * head run in order inside one task, so the dq/dk sums over rows and value heads (:194-198) have a fixed order. */
int FN(gdn_ref_bwd)(const gdn_ref_shape* sh, const REAL* q, const REAL* k, const REAL* v, const REAL* g,
                    const REAL* beta, const REAL* ckpt, const REAL* dy, const REAL* ds_out, REAL* dq, REAL* dk,
                    REAL* dv, REAL* dg, REAL* dbeta, REAL* ds0) {
  if (gdn_ref_check(sh) || !ckpt) return -1;
  const int N = gdn_ref_num_seqs(sh), Hk = sh->Hk, Hv = sh->Hv, Dk = sh->Dk, Dv = sh->Dv, C = sh->chunk;
  const int grp = Hv / Hk;
  const long SS = (long)Dv * Dk;
  int bad = 0;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int n = 0; n < N; ++n) {
    for (int hk = 0; hk < Hk; ++hk) {
      const FN(seq_t) sq = FN(seq_of)(sh, n);
      const int nch = (sq.len + C - 1) / C;
      REAL* st = (REAL*)malloc(sizeof(REAL) * (size_t)(C + 1) * Dk);
      REAL* del = (REAL*)malloc(sizeof(REAL) * (size_t)C);
      REAL* uu = (REAL*)malloc(sizeof(REAL) * (size_t)C);
      REAL* ds = (REAL*)malloc(sizeof(REAL) * (size_t)Dk);
      if (!st || !del || !uu || !ds) {
#pragma omp atomic write
        bad = 1;
        free(st), free(del), free(uu), free(ds);
        continue;
      }
      for (int t = 0; t < sq.len; ++t) {
        const long tok = sq.tok0 + t;
        for (int i = 0; i < Dk; ++i) dq[(tok * Hk + hk) * Dk + i] = dk[(tok * Hk + hk) * Dk + i] = 0;
      }
      for (int hv = hk * grp; hv < (hk + 1) * grp; ++hv) {
        for (int t = 0; t < sq.len; ++t) {
          const long tok = sq.tok0 + t;
          dg[tok * Hv + hv] = dbeta[tok * Hv + hv] = 0;
        }
        for (int r = 0; r < Dv; ++r) {
          const long row = (((long)n * Hv + hv) * Dv + r) * Dk;
          for (int i = 0; i < Dk; ++i) ds[i] = ds_out ? ds_out[row + i] : (REAL)0;
          for (int c = nch - 1; c >= 0; --c) {
            const int t0 = c * C, L = sq.len - t0 < C ? sq.len - t0 : C;
            const REAL* ck = ckpt + ((sq.slot0 + c) * Hv + hv) * SS + (long)r * Dk;
            for (int i = 0; i < Dk; ++i) st[i] = ck[i];
            for (int tt = 0; tt < L; ++tt) { /* recompute the chunk's states, :79-95 */
              const long tok = sq.tok0 + t0 + tt;
              const REAL* kt = k + (tok * Hk + hk) * Dk;
              const REAL gt = FN(decay)(sh, g, tok * Hv + hv), bt = beta[tok * Hv + hv];
              const REAL vt = v[(tok * Hv + hv) * Dv + r];
              REAL* a = st + (long)tt * Dk;
              REAL* b = a + Dk;
              REAL u = 0;
              for (int i = 0; i < Dk; ++i) {
                b[i] = a[i] * gt;
                u += b[i] * kt[i];
              }
              const REAL d = (vt - u) * bt;
              for (int i = 0; i < Dk; ++i) b[i] = b[i] + kt[i] * d;
              del[tt] = d;
              uu[tt] = u;
            }
            for (int tt = L - 1; tt >= 0; --tt) { /* reverse steps, :97-141 */
              const long tok = sq.tok0 + t0 + tt;
              const REAL* kt = k + (tok * Hk + hk) * Dk;
              const REAL* qt = q + (tok * Hk + hk) * Dk;
              REAL* dqt = dq + (tok * Hk + hk) * Dk;
              REAL* dkt = dk + (tok * Hk + hk) * Dk;
              const REAL gt = FN(decay)(sh, g, tok * Hv + hv), bt = beta[tok * Hv + hv];
              const long vr = (tok * Hv + hv) * Dv + r;
              const REAL vt = v[vr], dyt = dy[vr];
              const REAL* sp = st + (long)tt * Dk; /* S_prev */
              const REAL* sn = sp + Dk;            /* S_t */
              REAL dd = 0;
              for (int i = 0; i < Dk; ++i) {
                ds[i] += dyt * qt[i];
                dqt[i] += dyt * sn[i];
                dd += ds[i] * kt[i];
              }
              const REAL du = -bt * dd;
              REAL dgs = 0;
              for (int i = 0; i < Dk; ++i) {
                dkt[i] += ds[i] * del[tt] + du * (sp[i] * gt);
                ds[i] += du * kt[i];
                dgs += ds[i] * sp[i];
                ds[i] *= gt;
              }
              dv[vr] = bt * dd;
              dbeta[tok * Hv + hv] += dd * (vt - uu[tt]);
              dg[tok * Hv + hv] += dgs;
            }
          }
          if (ds0)
            for (int i = 0; i < Dk; ++i) ds0[row + i] = ds[i];
        }
        if (sh->g_is_log) /* d/da = g d/dg */
          for (int t = 0; t < sq.len; ++t) {
            const long tok = sq.tok0 + t;
            dg[tok * Hv + hv] *= FN(decay)(sh, g, tok * Hv + hv);
          }
      }
      free(st), free(del), free(uu), free(ds);
    }
  }
  return bad ? -1 : 0;
}

#undef FN
#undef CAT
#undef CAT2
