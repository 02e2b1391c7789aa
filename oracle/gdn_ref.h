/*
 * CPU restatement of quotebound's gated delta rule: the forward recurrence and its hand-written backward.
 *
 * TEST INFRASTRUCTURE ONLY. The kernels' results are compared with it: the parity tests, __graft_entry__.smoke()
 * and bench.py's CPU-baseline leg load it. The product (quotebound_amd, libqb_gdn.so) never links, loads or calls it, and has no
 * CPU fallback of any kind.
 *
 * What it restates (reference paths are relative to the quotebound checkout):
 *   forward, per value head, rows of the state S [Dv, Dk] independent       tests/gated_delta_ref.h:110-118
 *       S~ = g S;  u = S~ k;  delta = beta (v - u);  S = S~ + delta k^T;  y = S q
 *   GQA: value head hv reads key head hv / (Hv / Hk)                           tests/gated_delta_ref.h:18, 103
 *   chunk-start states, ckpt[c] = state after c*chunk steps, ckpt[0] = S0     src/delta_grad.cpp:172-181
 *   backward equations and their step order                                     src/delta_grad.cpp:14-18, 97-141
 *       dS += dy q^T; dq = S^T dy; dd = dS k; dk = dS^T delta + S~^T du; dv = beta dd; dbeta = dd (v - u);
 *       du = -beta dd; dS~ = dS + du k^T; dg = sum(dS~ * S_prev); dS_prev = g dS~
 *   reductions: dq, dk summed over rows, then over the value heads of a key head; dg, dbeta over rows
 *                                                                               src/delta_grad.cpp:194-198
 * Additions with no reference counterpart (documented in the build's design notes):
 *   g_is_log: g holds the log-decay a, g_t = exp(a_t), and the returned dg is d/da = g_t * d/dg_t.
 *   cu_seqlens: B == 1 and the T tokens are n_seqs packed sequences, each with its own initial and final state
 *   and its own chunking; defined as equal to independent calls per sequence.
 *
 * Layouts (row-major): q, k [B, T, Hk, Dk]; v, y, dy [B, T, Hv, Dv]; g, beta [B, T, Hv];
 * states [N, Hv, Dv, Dk] with N = B (or n_seqs); ckpt [NCtot, Hv, Dv, Dk], chunk slots of sequence n first.
 *
 * Parity status: every function here is pinned by tests/test_oracle.py (closed forms, finite differences,
 * autodiff through a plain-ops loop, and the committed golden vectors).
 */
#ifndef QB_GDN_REF_H
#define QB_GDN_REF_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gdn_ref_shape {
  int B, T, Hk, Hv, Dk, Dv;
  int chunk;             /* checkpoint stride in steps */
  int g_is_log;          /* 1: g holds log-decay */
  const int* cu_seqlens; /* host array of n_seqs + 1 offsets, or NULL */
  int n_seqs;
} gdn_ref_shape;

/* Number of chunk-start state slots the forward writes (sum over sequences of ceil(len / chunk)). */
long gdn_ref_num_chunks(const gdn_ref_shape* sh);
/* Number of sequences (B, or n_seqs with cu_seqlens). */
int gdn_ref_num_seqs(const gdn_ref_shape* sh);
/* 0 when the shape is usable, else -1. */
int gdn_ref_check(const gdn_ref_shape* sh);

/* s0 may be NULL (zero state); s_out and ckpt may be NULL. */
int gdn_ref_fwd_f32(const gdn_ref_shape* sh, const float* q, const float* k, const float* v, const float* g,
                    const float* beta, const float* s0, float* y, float* s_out, float* ckpt);
int gdn_ref_fwd_f64(const gdn_ref_shape* sh, const double* q, const double* k, const double* v, const double* g,
                    const double* beta, const double* s0, double* y, double* s_out, double* ckpt);

/* ckpt as the forward wrote it; ds_out may be NULL (zero cotangent on the final state); ds0 may be NULL. */
int gdn_ref_bwd_f32(const gdn_ref_shape* sh, const float* q, const float* k, const float* v, const float* g,
                    const float* beta, const float* ckpt, const float* dy, const float* ds_out, float* dq, float* dk,
                    float* dv, float* dg, float* dbeta, float* ds0);
int gdn_ref_bwd_f64(const gdn_ref_shape* sh, const double* q, const double* k, const double* v, const double* g,
                    const double* beta, const double* ckpt, const double* dy, const double* ds_out, double* dq,
                    double* dk, double* dv, double* dg, double* dbeta, double* ds0);

/* OpenMP threads the functions above use; set_threads(n <= 0) leaves the default. */
int gdn_ref_threads(void);
void gdn_ref_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
