// Design 2: the chunkwise WY/UT form on MFMA. Not built yet: every call is rejected with a clear error.
#include "gdn_kernels.h"

namespace qbgdn {

const char* chunk_supports(const Problem&) { return "the chunked design is not available in this build"; }
size_t chunk_ckpt_bytes(const Problem&) { return 0; }
size_t chunk_workspace_bytes(const Problem&) { return 0; }
const char* const kChunkFwdLaunches = "";
const char* const kChunkBwdLaunches = "";
hipError_t chunk_fwd(const Problem&, const FwdPtrs&, void*, hipStream_t, Tracer&) { return hipErrorNotSupported; }
hipError_t chunk_bwd(const Problem&, const BwdPtrs&, void*, hipStream_t, Tracer&) { return hipErrorNotSupported; }

}  // namespace qbgdn
