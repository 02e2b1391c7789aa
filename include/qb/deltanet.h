// The recurrence dispatcher with the reference's signature (src/deltanet.h:17-19, src/deltanet.cpp:49-61), on
// qb::array and the HIP kernels of qb_gdn.h.
//   q, k [B, T, Hk, Dk]; v [B, T, Hv, Dv]; g, beta [B, T, Hv]; state [B, Hv, Dv, Dk] float32.
// Per value head and step: S~ = g S; u = S~ k; delta = beta (v - u); S = S~ + delta k^T; y = S q. Arithmetic is
// float32; y comes back in q's dtype and the final state in float32, as in the reference. g is the decay factor
// and is never rounded to bfloat16. train selects the trainable op, whose forward is the same computation.
// Throws std::runtime_error naming the offending shapes when the kernels cannot run them.
#pragma once
#include <utility>

#include "qb/array.h"

namespace qb {

std::pair<array, array> gated_delta(const array& q, const array& k, const array& v, const array& g,
                                    const array& beta, const array& state, bool train = false);

// The forward keeping the state after every token: (y in q's dtype, states [B, T, Hv, Dv, Dk] float32, entry t
// the state after token t). It replaces the reference's rows pass, one gated_delta call per token
// (src/deltanet.cpp:101-117), whose states a draft decoder rolls back to (src/exact.cpp:152-162). It always runs
// the recurrent design, so Dk must be a multiple of 32 of at most 4096.
std::pair<array, array> gated_delta_rows(const array& q, const array& k, const array& v, const array& g,
                                         const array& beta, const array& state);

}  // namespace qb
