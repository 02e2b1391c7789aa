// The gated delta rule with its hand-written backward, with the reference's signatures (src/delta_grad.h:14-20,
// src/delta_grad.cpp:155-212), on qb::array and the HIP kernels of qb_gdn.h.
//   q, k [B, T, Hk, Dk]; v [B, T, Hv, Dv]; g, beta [B, T, Hv]; state [B, Hv, Dv, Dk].
#pragma once
#include <utility>
#include <vector>

#include "qb/array.h"

namespace qb {

// The forward of the trainable op: (y, final state). There is no autodiff graph to attach a vjp to here; a
// caller's training loop calls gated_delta_vjp with the same primals, as mx::custom_vjp does for the reference.
std::pair<array, array> gated_delta_trainable(const array& q, const array& k, const array& v, const array& g,
                                              const array& beta, const array& state);

// The backward alone: cotangents of (q, k, v, g, beta, state) given those of y and of the final state (an empty
// array is zero). Like the reference it first rebuilds the chunk-start states from the primals (64-step stride),
// then runs the backward kernels. Each cotangent comes back in its primal's dtype. Deterministic.
std::vector<array> gated_delta_vjp(const std::vector<array>& primals, const array& dy, const array& dstate);

}  // namespace qb
