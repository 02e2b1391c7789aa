/*
 * qb_gdn: the gated delta rule (Qwen3.5's Gated DeltaNet recurrence), forward and backward, as HIP kernels for
 * MI355X (gfx950) behind a C ABI.
 *
 * It replaces, on device buffers, the recurrence the reference runs through MLX and Metal:
 *   gated_delta(q, k, v, g, beta, state, train)          reference src/deltanet.h:17-19, src/deltanet.cpp:49-61
 *   gated_delta_trainable(q, k, v, g, beta, state)       reference src/delta_grad.h:14-16, src/delta_grad.cpp:201-212
 *   gated_delta_vjp(primals, dy, dstate)                 reference src/delta_grad.h:19-20, src/delta_grad.cpp:155-199
 * qb_gdn_fwd is the forward (mx::fast::gated_delta_update plus the chunk-start states the reference's vjp rebuilds
 * at src/delta_grad.cpp:172-181); qb_gdn_bwd is the vjp (the Metal kernel at :23-145 and the reductions at :194-198).
 * The C++ adapters with the reference's own signatures are in qb/deltanet.h and qb/delta_grad.h.
 *
 * Conventions (those of the reference's C library, src/constrain_capi.h:8-9): every call that can fail returns -1
 * and writes why into err (cut to errlen, NUL-terminated); nothing throws across the ABI. All data pointers are
 * caller-owned DEVICE buffers, row-major, in the layouts below. Work is queued on `stream` (a hipStream_t; NULL is
 * the default stream) and the calls return without waiting for it. The library keeps no mutable global state apart
 * from qb_gdn_bwd_static's per-GPU scratch array (and that array's address on each device, looked up once): the other
 * calls on different streams may overlap as long as they do not share output or workspace buffers.
 *
 * Layouts (N = B, or n_seqs with cu_seqlens; NC = chunk slots, see qb_gdn_num_chunks):
 *   q, k            [B, T, Hk, Dk]     dtype          key head of value head hv: hv / (Hv / Hk)
 *   v               [B, T, Hv, Dv]     dtype
 *   y, dy           [B, T, Hv, Dv]     out dtype      (dtype, or float32 with out_f32)
 *   g               [B, T, Hv]         float32        decay factor, or log-decay when g_is_log
 *   beta            [B, T, Hv]         dtype
 *   s0, s_out, ...  [N, Hv, Dv, Dk]    float32        state S (row = value index), as the reference's [B,Hv,Dv,Dk]
 *   ckpt            qb_gdn_ckpt_bytes  float32        starts with the chunk-start states [NC, Hv, Dv, Dk]
 *   dq, dk          [B, T, Hk, Dk]     out dtype; dv [B, T, Hv, Dv] out dtype; dbeta [B, T, Hv] out dtype
 *   dg              [B, T, Hv]         float32
 * Pointers to q, k and ckpt must be 16-byte aligned, the others aligned to their element size.
 *
 * Semantics per value head and step (reference tests/gated_delta_ref.h:110-118):
 *   S~ = g_t S;  u = S~ k_t;  delta = beta_t (v_t - u);  S = S~ + delta k_t^T;  y_t = S q_t
 * Arithmetic is float32 throughout; bf16 is an input/output format only.
 */
#ifndef QB_GDN_H
#define QB_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QB_GDN_MAX_SEQS 255 /* packed sequences per call */

typedef enum qb_dtype { QB_DTYPE_F32 = 0, QB_DTYPE_BF16 = 1 } qb_dtype;

typedef enum qb_gdn_design {
  QB_GDN_RECURRENT = 1, /* per state row: fp32 state in registers, wave-level reductions over Dk */
  QB_GDN_CHUNKED = 2    /* 64-token chunks in WY/UT form on bf16 MFMA with fp32 accumulation */
} qb_gdn_design;

typedef struct qb_gdn_desc {
  int32_t B, T, Hk, Hv, Dk, Dv;
  int32_t chunk;              /* checkpoint stride in steps: 64, the reference's kChunk (src/delta_grad.cpp:11) */
  int32_t dtype;              /* qb_dtype of q, k, v, beta (and of the outputs unless out_f32) */
  int32_t g_is_log;           /* 0: g is the decay factor and dg = dL/dg (the reference's convention);
                                 1: g is the log-decay a, g_t = exp(a_t), and dg = dL/da */
  int32_t design;             /* qb_gdn_design */
  int32_t out_f32;            /* 0: y, dy, dq, dk, dv, dbeta are in dtype (the reference returns y in q's dtype,
                                 src/deltanet.cpp:57, 60); 1: they are float32 whatever dtype is */
  const int32_t* cu_seqlens;  /* HOST array of n_seqs + 1 token offsets (0 .. T), or NULL. With it B must be 1 and
                                 the T tokens are n_seqs sequences, each with its own initial/final state and the
                                 state reset at each boundary: equal to one call per sequence. */
  int32_t n_seqs;
  void** trace_events;        /* Instrumentation, no reference counterpart; NULL for none. Caller-owned hipEvent_t
                                 handles: a call records trace_events[i] on its stream before its kernel launch i
                                 and trace_events[n] after its last launch (n = qb_gdn_launches), so the caller
                                 can time each kernel with hipEventElapsedTime. */
  int32_t n_trace_events;     /* at least qb_gdn_launches(...) + 1 when trace_events is set */
} qb_gdn_desc;

/* The library's version string. */
const char* qb_gdn_version(void);

/* 0 when the library supports desc, else -1 with the reason in err. Checks what qb_gdn_fwd / qb_gdn_bwd check. */
int qb_gdn_validate(const qb_gdn_desc* desc, char* err, int errlen);

/* Chunk slots: ceil(T / chunk) per sequence, summed. -1 on an invalid desc. */
int64_t qb_gdn_num_chunks(const qb_gdn_desc* desc);

/* Bytes of the residual buffer the forward writes and the backward reads (the chunk-start states, then what the
 * design keeps for its backward). 0 on an invalid desc. */
size_t qb_gdn_ckpt_bytes(const qb_gdn_desc* desc);

/* Bytes of scratch the forward and the backward need (may be 0; the pointer may then be NULL). The contents do
 * not need to survive between calls. 0 on an invalid desc. */
size_t qb_gdn_workspace_bytes(const qb_gdn_desc* desc);

/* The main kernels a call launches, in order, as its trace events time them (the small follow-up passes are timed
 * with the kernel before them: the chunked backward's dq/dk sum for short sequences, its gate-parameter sums with the
 * fused prologue, and its exact dL/dg replay where g is the decay factor): their count is returned
 * and their names written comma-separated into names (cut to len; may be NULL). which: 0 for qb_gdn_fwd, 1 for
 * qb_gdn_bwd. -1 on an invalid desc. */
int qb_gdn_launches(const qb_gdn_desc* desc, int which, char* names, int len);

/* Forward. s0 may be NULL (zero initial state); s_out may be NULL; ckpt may be NULL when no backward follows. */
int qb_gdn_fwd(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g, const void* beta,
               const float* s0, void* y, float* s_out, float* ckpt, void* workspace, void* stream, char* err,
               int errlen);

/* Forward that also keeps the state after every token, for decoding that may roll back (exact drafts): replaces
 * the reference's rows pass, one gated_delta call per token keeping each step's state (src/deltanet.cpp:101-117;
 * RowStates, src/model.h:80-86; keep_rows, src/exact.cpp:152-162). row_states [tokens, Hv, Dv, Dk] float32, where
 * tokens is B*T (or the packed total): entry t is the state after token t. Always runs the recurrent design, whatever
 * desc->design says (the shape must suit it: Dk a multiple of 32 of at most 4096), so no ckpt or workspace is taken. */
int qb_gdn_fwd_rows(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g,
                    const void* beta, const float* s0, void* y, float* row_states, void* stream, char* err,
                    int errlen);

/* Backward from the forward's ckpt: the cotangents of (q, k, v, g, beta, s0) given dy and ds_out (the cotangent of
 * the final state; NULL is zero). ds0 may be NULL. Deterministic: sums run in a fixed order, no atomics. ckpt must
 * come from a forward of the same desc, design included (past the states each design keeps its own residual). */
int qb_gdn_bwd(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g,
               const void* beta, const float* ckpt, const void* dy, const float* ds_out, void* dq, void* dk, void* dv,
               float* dg, void* dbeta, float* ds0, void* workspace, void* stream, char* err, int errlen);

/* Size of the device array qb_gdn_bwd_static uses as its workspace, per GPU: 257 MiB, which holds the chunked
 * design's workspace (the chunk-end state cotangents and 8 bytes per chunk and value head) up to
 * NC * Hv * Dv * Dk = 2^26 (the 4B layer shape at T = 4096 uses half of it, the 9B shape three quarters). */
#define QB_GDN_STATIC_SCRATCH_BYTES (257u << 20)

/* qb_gdn_bwd without a workspace argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. Its workspace is
 * a file-scope device array of QB_GDN_STATIC_SCRATCH_BYTES that each GPU the library runs on holds until the
 * process ends; a desc whose qb_gdn_workspace_bytes exceeds that is refused with -1 and the reason in err, before any
 * GPU work. It calls no hipMalloc, hipFree or allocating routine. The first call on a device looks up that device's
 * address of the array (with the device current), which may load the library's device code: make that first call
 * outside any graph capture. Later calls only launch kernels on the stream (no memset, no copy), so they may be
 * captured into a HIP graph and replayed. Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (on different streams, or unordered across host threads) race on it and must not be issued. Nothing in
 * the array needs to start at zero (the backward writes every byte of its workspace before reading it), and it keeps
 * the last call's contents. Otherwise as qb_gdn_bwd, with the same outputs bit for bit. */
int qb_gdn_bwd_static(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g,
                      const void* beta, const float* ckpt, const void* dy, const float* ds_out, void* dq, void* dk,
                      void* dv, float* dg, void* dbeta, float* ds0, void* stream, char* err, int errlen);

/* The layer's pointwise neighbours of the recurrence, each one pass over its rows (reference src/deltanet.cpp). They
 * read B, T, Hk, Hv, Dk, Dv and dtype from desc (the other fields are not used; the prologue needs Dk, the epilogue
 * Dv, of 64, 128 or 256, and Hv at most 256)
 * and take the activations in dtype and the parameters in float32. With bf16 activations each op's output is
 * rounded to bf16 where the reference's op rounds it; arithmetic inside an op is float32. The backward entry points
 * are float32 inside with one rounding of each output, and sum the parameter gradients over tokens in a fixed order
 * (deterministic). Pointers to the row tensors (q_raw, k_raw, q, k, y, z, o, dout and their cotangents) and to
 * norm_w must be 16-byte aligned, the others aligned to their element size. */

/* Scratch the neighbours' backward entry points need (the per-block partial sums); 0 on an invalid desc. */
size_t qb_gdn_neighbours_workspace_bytes(const qb_gdn_desc* desc);

/* Prologue, before qb_gdn_fwd (src/deltanet.cpp:22-33, 94-100): q = s_q rms_norm(q_raw) and k = s_k rms_norm(k_raw)
 * (no weight, eps 1e-6; s_q = 1/Dk and s_k = Dk^-1/2 in dtype), beta = sigmoid(b), and the log-decay
 * -exp(a_log) softplus(a + dt_bias), the g of qb_gdn_fwd with g_is_log = 1 (the reference's compute_g takes its
 * exp). q_raw, k_raw, q, k [B, T, Hk, Dk]; a, b, beta [B, T, Hv] in dtype; a_log, dt_bias [Hv]; log_decay
 * [B, T, Hv] float32. */
int qb_gdn_prologue_fwd(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* a, const void* b,
                        const float* a_log, const float* dt_bias, void* q, void* k, void* beta, float* log_decay,
                        void* stream, char* err, int errlen);

/* Its backward: from the cotangents of q, k, beta (dtype) and of the log-decay (float32), those of q_raw, k_raw, a,
 * b (dtype) and of a_log, dt_bias ([Hv] float32, summed over every token). */
int qb_gdn_prologue_bwd(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* a, const void* b,
                        const float* a_log, const float* dt_bias, const void* dq, const void* dk, const void* dbeta,
                        const float* dlog_decay, void* dq_raw, void* dk_raw, void* da, void* db, float* da_log,
                        float* ddt_bias, void* workspace, void* stream, char* err, int errlen);

/* qb_gdn_prologue_fwd and qb_gdn_fwd in one: the prologue runs inside the forward's first kernel, which reads q_raw,
 * k_raw, a and b in place of q, k, g and beta, forms those exactly as qb_gdn_prologue_fwd does (bit for bit), writes
 * them (q, k, beta, log_decay as there: the backward reads them) and goes on as qb_gdn_fwd with g = log_decay. It saves
 * the separate pass over q_raw and k_raw and its launch (reference src/deltanet.cpp:94-100 feeding
 * gated_delta_update, :101-117). The chunked design only: desc->design QB_GDN_CHUNKED, dtype bf16, g_is_log = 1 (the
 * prologue emits the log-decay); s0, s_out and ckpt as for qb_gdn_fwd. */
int qb_gdn_fwd_prologue(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* v, const void* a,
                        const void* b, const float* a_log, const float* dt_bias, const float* s0, void* q, void* k,
                        void* beta, float* log_decay, void* y, float* s_out, float* ckpt, void* workspace,
                        void* stream, char* err, int errlen);

/* qb_gdn_bwd and qb_gdn_prologue_bwd in one, after qb_gdn_fwd_prologue: the prologue's backward runs at the end of
 * the backward's last kernel, which rounds the cotangents of q, k and beta to bf16 as qb_gdn_prologue_bwd would read
 * them and turns them, with that of the log-decay, into those of q_raw, k_raw, a, b (bf16) and of a_log, dt_bias
 * ([Hv] float32, summed over every token: per (chunk, value head) in the kernel, then over chunks in order, a
 * fixed order but not qb_gdn_prologue_bwd's). q, k, beta, log_decay and ckpt are what qb_gdn_fwd_prologue wrote.
 * It saves the separate pass's reads of dq, dk, q_raw, k_raw and its launch; dq_raw and dk_raw leave as 16-byte
 * row stores. The chunked design only: desc->design QB_GDN_CHUNKED, dtype bf16, out_f32 = 0, g_is_log = 1. ds_out
 * and ds0 as for qb_gdn_bwd. */
int qb_gdn_bwd_prologue(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* a, const void* b,
                        const float* a_log, const float* dt_bias, const void* q, const void* k, const void* v,
                        const void* beta, const float* log_decay, const float* ckpt, const void* dy,
                        const float* ds_out, void* dq_raw, void* dk_raw, void* dv, void* da, void* db, float* da_log,
                        float* ddt_bias, float* ds0, void* workspace, void* stream, char* err, int errlen);

/* Epilogue, after qb_gdn_fwd (src/deltanet.cpp:35-45, 122, the gated RMSNorm): o = silu(z) rms_norm(y, norm_w, eps).
 * y, z, o [B, T, Hv, Dv] in dtype; norm_w [Dv] float32. */
int qb_gdn_epilogue_fwd(const qb_gdn_desc* desc, const void* y, const void* z, const float* norm_w, float eps, void* o,
                        void* stream, char* err, int errlen);

/* Its backward: from the cotangent of o, those of y and z (dtype) and of norm_w ([Dv] float32, summed over every
 * row). */
int qb_gdn_epilogue_bwd(const qb_gdn_desc* desc, const void* y, const void* z, const float* norm_w, float eps,
                        const void* dout, void* dy, void* dz, float* dnorm_w, void* workspace, void* stream, char* err,
                        int errlen);

#ifdef __cplusplus
}
#endif
#endif
