// Chunked design: the host side. The forward is prep (T, G per chunk) then the sequential state pass (states,
// y, final state); the backward is the reverse state pass (dv, ds0 and each chunk's end-state cotangent) then the
// per-chunk gradient kernel (dq, dk, dg, dbeta), and, when g is given as the decay factor, the exact dL/dg at tiny
// factors.
#include "chunk_kernels.h"
#include "gdn_kernels.h"

namespace qbgdn {
namespace {

ChunkLayout layout_of(const Problem& p) { return ChunkLayout{p.NC, p.Hv, p.Dv, p.Dk}; }

size_t extras_bytes(const Problem& p) { return layout_of(p).tiles_bytes(); }
size_t dsend_bytes(const Problem& p) { return size_t(p.NC) * p.Hv * p.Dv * p.Dk * 4; }
// The fused prologue backward's per-(chunk slot, value head) sums, after dSend.
size_t gate_part_bytes(const Problem& p) { return (size_t(p.NC) * p.Hv * 2 * 4 + 255) & ~size_t(255); }

// The current device's compute-unit count; 256 (MI355X) when it cannot be read, as with no device (host-only
// sizing calls).
int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  return cus;
}

// Short sequences: when the (chunk slot, value head) pairs fit one per CU of the current device (NC * Hv <= CUs), the
// gradient kernel takes each value head of a GQA group as a work item of its own, so that the group's heads run side
// by side rather than in turn, and a second pass sums their dq and dk in order. Past that, its items already fill
// the device and the heads run in turn with dq, dk summed in registers. The workspace is sized by the same rule on
// the device current at sizing time.
bool split_grads(const Problem& p) { return p.Hv > p.Hk && int64_t(p.NC) * p.Hv <= device_cus(); }
size_t dqk_part_bytes(const Problem& p) { return split_grads(p) ? size_t(p.NC) * p.Hv * 2 * 64 * p.Dk * 4 : 0; }

// State rows per block of the state passes: 16, or 32 when the 16-row blocks (one resident per CU) would take more
// than one round of the device, so that each block's per-chunk loads of k, q and the tile serve twice the rows.
int state_rows(const Problem& p) { return int64_t(p.N) * p.Hv * (p.Dv / 16) > device_cus() ? 32 : 16; }

ChunkArgs base_args(const Problem& p) {
  ChunkArgs a{};
  a.lay = layout_of(p);
  a.Hk = p.Hk, a.Hv = p.Hv, a.Dv = p.Dv, a.g_is_log = p.g_is_log;
  a.nblk = p.Dv / state_rows(p);
  a.N = p.N;
  a.tab = p.tab;
  return a;
}

// The tiles sit after the states in ckpt, or at the start of the workspace when there is no ckpt.
void place_extras(const Problem&, ChunkArgs& a, float* ckpt, void* ws) {
  a.tiles = reinterpret_cast<Tile*>(ckpt ? ckpt + a.lay.states_elems() : static_cast<float*>(ws));
}

}  // namespace

const char* const kChunkFwdLaunches = "chunk_prep,chunk_fwd";
const char* const kChunkBwdLaunches = "chunk_bwd_state,chunk_bwd_grads";

const char* chunk_supports(const Problem& p) {
  if (!p.in_bf16) return "the chunked design needs bf16 inputs (use the recurrent design for float32)";
  if (p.Dk != 128) return "the chunked design needs Dk of 128";
  if (p.Dv % 32) return "the chunked design needs Dv a multiple of 32";
  if (p.NC * p.Hv > (int64_t(1) << 30) || int64_t(p.N) * p.Hv * (p.Dv / 16) > (int64_t(1) << 30))
    return "problem too large for the chunked design's grid";
  return nullptr;
}

size_t chunk_ckpt_bytes(const Problem& p) { return layout_of(p).bytes(); }

size_t chunk_workspace_bytes(const Problem& p) {
  const size_t a = dsend_bytes(p) + gate_part_bytes(p) + dqk_part_bytes(p), b = extras_bytes(p);
  return a > b ? a : b;
}

namespace {

hipError_t fwd_impl(const Problem& p, const PrologueIn* pro, const FwdPtrs& f, void* ws, hipStream_t s, Tracer& tr) {
  ChunkArgs a = base_args(p);
  a.q = static_cast<const bf16_t*>(f.q);
  a.k = static_cast<const bf16_t*>(f.k);
  a.v = static_cast<const bf16_t*>(f.v);
  a.beta = static_cast<const bf16_t*>(f.beta);
  a.g = f.g;
  a.s0 = f.s0;
  a.y = f.y;
  a.s_out = f.s_out;
  a.ckpt = f.ckpt;
  place_extras(p, a, f.ckpt, ws);
  if (pro) {
    a.pro = ChunkArgs::Prologue{static_cast<const bf16_t*>(pro->q_raw), static_cast<const bf16_t*>(pro->k_raw),
                                static_cast<const bf16_t*>(pro->a),     static_cast<const bf16_t*>(pro->b),
                                pro->a_log,                             pro->dt_bias,
                                pro->scale_q,                           pro->scale_k,
                                static_cast<bf16_t*>(pro->q),           static_cast<bf16_t*>(pro->k),
                                static_cast<bf16_t*>(pro->beta),        pro->log_decay};
  }
  tr.mark();
  hipError_t e = launch_chunk_prep(a, s, pro != nullptr);
  if (e != hipSuccess) return e;
  tr.mark();
  e = launch_chunk_fwd(a, p.out_bf16, s);
  tr.mark();
  return e;
}

}  // namespace

hipError_t chunk_fwd(const Problem& p, const FwdPtrs& f, void* ws, hipStream_t s, Tracer& tr) {
  return fwd_impl(p, nullptr, f, ws, s, tr);
}

hipError_t chunk_fwd_prologue(const Problem& p, const PrologueIn& pro, const FwdPtrs& f, void* ws, hipStream_t s,
                              Tracer& tr) {
  if (!p.g_is_log || !p.in_bf16) return hipErrorInvalidValue;
  return fwd_impl(p, &pro, f, ws, s, tr);
}

namespace {

hipError_t bwd_impl(const Problem& p, const PrologueGradIn* pro, const BwdPtrs& b, void* ws, hipStream_t s,
                    Tracer& tr) {
  ChunkArgs a = base_args(p);
  a.q = static_cast<const bf16_t*>(b.q);
  a.k = static_cast<const bf16_t*>(b.k);
  a.v = static_cast<const bf16_t*>(b.v);
  a.beta = static_cast<const bf16_t*>(b.beta);
  a.g = b.g;
  a.ckpt = const_cast<float*>(b.ckpt);
  place_extras(p, a, a.ckpt, nullptr);
  a.dy = b.dy;
  a.ds_out = b.ds_out;
  a.dq = b.dq;
  a.dk = b.dk;
  a.dv = b.dv;
  a.dg = b.dg;
  a.dbeta = b.dbeta;
  a.ds0 = b.ds0;
  a.dsend = static_cast<float*>(ws);
  if (split_grads(p))
    a.dqk_part = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + dsend_bytes(p) + gate_part_bytes(p));
  if (pro) {
    a.pro.q_raw = static_cast<const bf16_t*>(pro->q_raw), a.pro.k_raw = static_cast<const bf16_t*>(pro->k_raw);
    a.pro.a = static_cast<const bf16_t*>(pro->a), a.pro.b = static_cast<const bf16_t*>(pro->b);
    a.pro.a_log = pro->a_log, a.pro.dt_bias = pro->dt_bias;
    a.pro.scale_q = pro->scale_q, a.pro.scale_k = pro->scale_k;
    a.pro.da = static_cast<bf16_t*>(pro->da), a.pro.db = static_cast<bf16_t*>(pro->db);
    a.pro.part = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + dsend_bytes(p));
    a.dq = pro->dq_raw, a.dk = pro->dk_raw;
  }
  tr.mark();
  hipError_t e = launch_chunk_bwd_state(a, p.out_bf16, s);
  if (e != hipSuccess) return e;
  tr.mark();
  e = launch_chunk_bwd_grads(a, p.out_bf16, s, pro != nullptr);
  // The follow-up passes are timed with the gradient kernel. With the prologue, the sum pass also does the
  // normalisation's backward.
  if (e == hipSuccess && a.dqk_part) e = launch_chunk_dqk_sum(a, p.out_bf16, s, pro != nullptr);
  if (e == hipSuccess && pro) e = launch_chunk_gate_sums(a, pro->da_log, pro->ddt_bias, s);
  // With g given as the factor, dL/dg at tiny or zero factors comes from an exact replay (chunk_dgfix.hip); chunks
  // without one return at once.
  if (e == hipSuccess && !p.g_is_log) e = launch_chunk_dgfix(a, p.out_bf16, s);
  tr.mark();
  return e;
}

}  // namespace

hipError_t chunk_bwd(const Problem& p, const BwdPtrs& b, void* ws, hipStream_t s, Tracer& tr) {
  return bwd_impl(p, nullptr, b, ws, s, tr);
}

hipError_t chunk_bwd_prologue(const Problem& p, const PrologueGradIn& pro, const BwdPtrs& b, void* ws,
                              hipStream_t s, Tracer& tr) {
  if (!p.g_is_log || !p.in_bf16 || !p.out_bf16) return hipErrorInvalidValue;
  return bwd_impl(p, &pro, b, ws, s, tr);
}

}  // namespace qbgdn
