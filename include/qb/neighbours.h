// The DeltaNet layer's pointwise neighbours of the recurrence (reference src/deltanet.cpp:22-45, 94-100, 122), on
// qb::array and the HIP kernels of qb_gdn.h. Activations (q_raw, k_raw, a, b, y, z and their cotangents) run in
// bfloat16 when all of a call's activations are bfloat16, else in float32, with the reference's bf16 roundings in
// the former case; parameters (a_log, dt_bias, norm_w) and the log-decay are float32. The prologue needs Dk, the
// epilogue Dv, of 64, 128 or 256. Throws std::runtime_error naming the shapes when they do not fit. The prologue
// also comes fused into the recurrence (deltanet_prologue_recurrence and its vjp).
#pragma once
#include "qb/array.h"

namespace qb {

// Before the recurrence: q = rms_norm(q_raw) / Dk, k = rms_norm(k_raw) / sqrt(Dk) (no weight, eps 1e-6),
// beta = sigmoid(b), log_decay = -exp(a_log) * softplus(a + dt_bias) (compute_g before its exp: exp(log_decay) is
// gated_delta's g, and qb_gdn_fwd takes log_decay itself with g_is_log = 1). q_raw, k_raw [B, T, Hk, Dk];
// a, b [B, T, Hv]; a_log, dt_bias [Hv].
struct Prologue {
  array q, k, beta, log_decay;
};
Prologue deltanet_prologue(const array& q_raw, const array& k_raw, const array& a, const array& b,
                           const array& a_log, const array& dt_bias);

// Its backward: the cotangents of (q_raw, k_raw, a, b) in the activations' dtype and of (a_log, dt_bias) in
// float32, summed over tokens in a fixed order, given those of (q, k, beta, log_decay).
struct PrologueGrads {
  array dq_raw, dk_raw, da, db, da_log, ddt_bias;
};
PrologueGrads deltanet_prologue_vjp(const array& q_raw, const array& k_raw, const array& a, const array& b,
                                    const array& a_log, const array& dt_bias, const array& dq, const array& dk,
                                    const array& dbeta, const array& dlog_decay);

// After the recurrence: o = silu(z) * rms_norm(y, norm_w, eps). y, z [B, T, Hv, Dv]; norm_w [Dv].
array deltanet_epilogue(const array& y, const array& z, const array& norm_w, float eps);

// Its backward: the cotangents of y, z (activations' dtype) and norm_w (float32) given that of o.
struct EpilogueGrads {
  array dy, dz, dnorm_w;
};
EpilogueGrads deltanet_epilogue_vjp(const array& y, const array& z, const array& norm_w, float eps,
                                    const array& dout);

// The prologue inside the recurrence (qb_gdn_fwd_prologue): deltanet_prologue and then the gated delta rule on its
// outputs, with the log-decay as g's log (src/deltanet.cpp:94-101 feeding gated_delta at :111), in one call whose
// results equal those two steps' bit for bit; it saves the prologue's separate pass over q_raw and k_raw and its
// launch. y in bfloat16 and the final state in float32; q, k, beta, log_decay as deltanet_prologue returns them.
// The chunked design's shapes: bfloat16 activations (q_raw, k_raw [B, T, Hk, 128], v [B, T, Hv, Dv] with Dv a
// multiple of 32, a, b [B, T, Hv]); a_log, dt_bias [Hv] float32; state [B, Hv, Dv, Dk] float32, or empty for zeros.
struct PrologueRecurrence {
  array y, state, q, k, beta, log_decay;
};
PrologueRecurrence deltanet_prologue_recurrence(const array& q_raw, const array& k_raw, const array& v,
                                                const array& a, const array& b, const array& a_log,
                                                const array& dt_bias, const array& state);

// Its backward in gated_delta_vjp's form (qb_gdn_bwd_prologue): the forward runs again for the chunk-start states,
// then the backward, with the prologue's backward at the end of its last kernel. The cotangents of q_raw, k_raw, v,
// a, b in bfloat16, of a_log and dt_bias ([Hv] float32, summed over tokens in a fixed order: per chunk, then over
// chunks) and of state (float32), given dy (bfloat16 [B, T, Hv, Dv]) and dstate (empty is zero).
struct PrologueRecurrenceGrads {
  array dq_raw, dk_raw, dv, da, db, da_log, ddt_bias, dstate;
};
PrologueRecurrenceGrads deltanet_prologue_recurrence_vjp(const array& q_raw, const array& k_raw, const array& v,
                                                         const array& a, const array& b, const array& a_log,
                                                         const array& dt_bias, const array& state, const array& dy,
                                                         const array& dstate);

}  // namespace qb
