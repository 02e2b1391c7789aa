// The C ABI of include/qb_gdn.h: validates a descriptor, resolves it into a Problem and dispatches to the design's
// kernels. Every entry point catches everything; failures return -1 with the reason in err (the convention of
// reference src/constrain_capi.h:8-9). No mutable global state.
#include "qb_gdn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <string>

#include "gdn_kernels.h"
#include "neighbours.h"

namespace {

using qbgdn::Problem;

void set_err(char* err, int errlen, const std::string& what) {
  if (!err || errlen <= 0) return;
  std::strncpy(err, what.c_str(), size_t(errlen) - 1);
  err[errlen - 1] = '\0';
}

template <class F>
int guarded(char* err, int errlen, F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    set_err(err, errlen, e.what());
  } catch (...) {
    set_err(err, errlen, "unknown error");
  }
  return -1;
}

std::string shape_of(const qb_gdn_desc& d) {
  char buf[160];
  std::snprintf(buf, sizeof buf, "(B %d, T %d, Hk %d, Hv %d, Dk %d, Dv %d, chunk %d)", d.B, d.T, d.Hk, d.Hv, d.Dk,
                d.Dv, d.chunk);
  return buf;
}

// Resolves and checks desc; returns an empty string when usable, else the reason.
std::string resolve(const qb_gdn_desc* d, Problem& p) {
  if (!d) return "gated delta: null descriptor";
  const std::string sh = shape_of(*d);
  if (d->B < 1 || d->T < 0 || d->Hk < 1 || d->Hv < 1 || d->Dk < 1 || d->Dv < 1)
    return "gated delta: sizes must be positive " + sh;
  if (d->Hv % d->Hk)
    return "gated delta: value heads must be a multiple of key heads " + sh;
  if (d->Dk % 32) return "gated delta: needs Dk a multiple of 32 " + sh;
  if (d->chunk != qbgdn::kChunk) return "gated delta: the checkpoint stride must be 64 " + sh;
  if (d->dtype != QB_DTYPE_F32 && d->dtype != QB_DTYPE_BF16) return "gated delta: dtype must be f32 or bf16";
  if (d->g_is_log != 0 && d->g_is_log != 1) return "gated delta: g_is_log must be 0 or 1";
  if (d->design != QB_GDN_RECURRENT && d->design != QB_GDN_CHUNKED)
    return "gated delta: design must be 1 (recurrent) or 2 (chunked)";
  if (d->out_f32 != 0 && d->out_f32 != 1) return "gated delta: out_f32 must be 0 or 1";
  const int64_t BT = int64_t(d->B) * d->T;
  // Element counts must fit the kernels' 64-bit offsets with room; token counts a 32-bit grid dimension.
  if (BT > (int64_t(1) << 31) || int64_t(d->Hv) * d->Dv * d->Dk > (int64_t(1) << 31))
    return "gated delta: problem too large " + sh;
  p = Problem{};
  p.B = d->B, p.T = d->T, p.Hk = d->Hk, p.Hv = d->Hv, p.Dk = d->Dk, p.Dv = d->Dv;
  p.in_bf16 = d->dtype == QB_DTYPE_BF16;
  p.out_bf16 = p.in_bf16 && !d->out_f32;
  p.g_is_log = d->g_is_log;
  p.BT = BT;
  const int64_t per = (d->T + qbgdn::kChunk - 1) / qbgdn::kChunk;
  if (d->cu_seqlens) {
    if (d->B != 1) return "gated delta: packed sequences need B == 1 " + sh;
    if (d->n_seqs < 1 || d->n_seqs > QB_GDN_MAX_SEQS)
      return "gated delta: n_seqs must be in [1, " + std::to_string(QB_GDN_MAX_SEQS) + "], got " +
             std::to_string(d->n_seqs);
    const int32_t* cu = d->cu_seqlens;
    if (cu[0] != 0 || cu[d->n_seqs] != d->T)
      return "gated delta: cu_seqlens must run from 0 to T " + sh;
    p.tab.n = d->n_seqs;
    int64_t slots = 0;
    for (int i = 0; i < d->n_seqs; ++i) {
      if (cu[i + 1] < cu[i]) return "gated delta: cu_seqlens must not decrease";
      p.tab.tok0[i] = cu[i];
      p.tab.slot0[i] = int32_t(slots);
      slots += (cu[i + 1] - cu[i] + qbgdn::kChunk - 1) / qbgdn::kChunk;
    }
    p.tab.tok0[d->n_seqs] = cu[d->n_seqs];
    p.tab.slot0[d->n_seqs] = int32_t(slots);
    int order[QB_GDN_MAX_SEQS];
    for (int i = 0; i < d->n_seqs; ++i) order[i] = i;
    std::stable_sort(order, order + d->n_seqs, [&](int x, int y) { return cu[x + 1] - cu[x] > cu[y + 1] - cu[y]; });
    for (int i = 0; i < d->n_seqs; ++i) p.tab.longest[i] = uint8_t(order[i]);
    p.N = d->n_seqs;
    p.NC = slots;
  } else {
    p.tab.n = 0;
    p.tab.T = d->T;
    p.tab.nc = int32_t(per);
    p.N = d->B;
    p.NC = per * d->B;
  }
  const char* why = d->design == QB_GDN_RECURRENT ? qbgdn::rec_supports(p) : qbgdn::chunk_supports(p);
  if (why) return std::string("gated delta: ") + why + " " + sh;
  return {};
}

bool aligned(const void* ptr, size_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

std::string check_ptr(const char* name, const void* ptr, bool required, size_t align) {
  if (!ptr) return required ? std::string("gated delta: ") + name + " is null" : std::string();
  if (!aligned(ptr, align))
    return std::string("gated delta: ") + name + " must be " + std::to_string(align) + "-byte aligned";
  return {};
}

struct PtrCheck {
  const char* name;
  const void* ptr;
  bool req;
  size_t align;
};

template <size_t N>
std::string check_all(const PtrCheck (&c)[N]) {
  for (const auto& x : c) {
    std::string why = check_ptr(x.name, x.ptr, x.req, x.align);
    if (!why.empty()) return why;
  }
  return {};
}

size_t ckpt_bytes(const qb_gdn_desc* d, const Problem& p) {
  return d->design == QB_GDN_RECURRENT ? qbgdn::rec_ckpt_bytes(p) : qbgdn::chunk_ckpt_bytes(p);
}

size_t ws_bytes(const qb_gdn_desc* d, const Problem& p) {
  return d->design == QB_GDN_RECURRENT ? qbgdn::rec_workspace_bytes(p) : qbgdn::chunk_workspace_bytes(p);
}

qbgdn::Tracer tracer_of(const qb_gdn_desc* d, hipStream_t s) {
  qbgdn::Tracer t;
  t.ev = d->trace_events;
  t.n = d->trace_events ? d->n_trace_events : 0;
  t.s = s;
  return t;
}

int count_names(const char* names) {
  if (!*names) return 0;
  int n = 1;
  for (const char* c = names; *c; ++c) n += *c == ',';
  return n;
}

std::string hip_fail(const char* what, hipError_t e) {
  return std::string("gated delta: ") + what + " failed: " + hipGetErrorString(e);
}

}  // namespace

extern "C" {

const char* qb_gdn_version(void) { return "qb_gdn 0.1 (gfx950)"; }

int qb_gdn_validate(const qb_gdn_desc* desc, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    Problem p;
    const std::string why = resolve(desc, p);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    return 0;
  });
}

int qb_gdn_launches(const qb_gdn_desc* desc, int which, char* names, int len) {
  try {
    Problem p;
    if (!resolve(desc, p).empty() || (which != 0 && which != 1)) return -1;
    const bool rec = desc->design == QB_GDN_RECURRENT;
    const char* list = which == 0 ? (rec ? qbgdn::kRecFwdLaunches : qbgdn::kChunkFwdLaunches)
                                  : (rec ? qbgdn::kRecBwdLaunches : qbgdn::kChunkBwdLaunches);
    set_err(names, len, list);
    return count_names(list);
  } catch (...) {
    return -1;
  }
}

int64_t qb_gdn_num_chunks(const qb_gdn_desc* desc) {
  try {
    Problem p;
    return resolve(desc, p).empty() ? p.NC : -1;
  } catch (...) {
    return -1;
  }
}

size_t qb_gdn_ckpt_bytes(const qb_gdn_desc* desc) {
  try {
    Problem p;
    return resolve(desc, p).empty() ? ckpt_bytes(desc, p) : 0;
  } catch (...) {
    return 0;
  }
}

size_t qb_gdn_workspace_bytes(const qb_gdn_desc* desc) {
  try {
    Problem p;
    return resolve(desc, p).empty() ? ws_bytes(desc, p) : 0;
  } catch (...) {
    return 0;
  }
}

int qb_gdn_fwd(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g, const void* beta,
               const float* s0, void* y, float* s_out, float* ckpt, void* workspace, void* stream, char* err,
               int errlen) {
  return guarded(err, errlen, [&] {
    Problem p;
    std::string why = resolve(desc, p);
    const size_t el = p.in_bf16 ? 2 : 4, eo = p.out_bf16 ? 2 : 4;
    const bool any = p.BT > 0;
    const struct {
      const char* name;
      const void* ptr;
      bool req;
      size_t align;
    } ptrs[] = {{"q", q, any, 16},           {"k", k, any, 16},         {"v", v, any, el},
                {"g", g, any, 4},            {"beta", beta, any, el},   {"s0", s0, false, 4},
                {"y", y, any, eo},           {"s_out", s_out, false, 4}, {"ckpt", ckpt, false, 16},
                {"workspace", workspace, why.empty() && any && ws_bytes(desc, p) > 0, 16}};
    for (const auto& c : ptrs)
      if (why.empty()) why = check_ptr(c.name, c.ptr, c.req, c.align);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    const qbgdn::FwdPtrs a{q, k, v, g, beta, s0, y, s_out, ckpt};
    hipStream_t s = static_cast<hipStream_t>(stream);
    qbgdn::Tracer tr = tracer_of(desc, s);
    const hipError_t e = desc->design == QB_GDN_RECURRENT ? qbgdn::rec_fwd(p, a, workspace, s, tr)
                                                          : qbgdn::chunk_fwd(p, a, workspace, s, tr);
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("forward launch", e));
      return -1;
    }
    return 0;
  });
}

int qb_gdn_fwd_rows(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g,
                    const void* beta, const float* s0, void* y, float* row_states, void* stream, char* err,
                    int errlen) {
  return guarded(err, errlen, [&] {
    if (!desc) {
      set_err(err, errlen, "gated delta: null descriptor");
      return -1;
    }
    qb_gdn_desc d = *desc;
    d.design = QB_GDN_RECURRENT;
    Problem p;
    std::string why = resolve(&d, p);
    const size_t el = p.in_bf16 ? 2 : 4, eo = p.out_bf16 ? 2 : 4;
    const bool any = why.empty() && p.BT > 0;
    const PtrCheck c[] = {{"q", q, any, 16},       {"k", k, any, 16},     {"v", v, any, el},
                          {"g", g, any, 4},        {"beta", beta, any, el}, {"s0", s0, false, 4},
                          {"y", y, any, eo},       {"row_states", row_states, any, 16}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    qbgdn::FwdPtrs a{q, k, v, g, beta, s0, y, nullptr, nullptr};
    a.rows = row_states;
    hipStream_t s = static_cast<hipStream_t>(stream);
    qbgdn::Tracer tr = tracer_of(&d, s);
    const hipError_t e = qbgdn::rec_fwd(p, a, nullptr, s, tr);
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("forward launch", e));
      return -1;
    }
    return 0;
  });
}

}  // extern "C"

namespace {

// The backward's scratch for callers that cannot allocate (qb_gdn_bwd_static): one array per GPU, which each GPU
// the library runs on holds until the process ends. In host code the name `scratch` is not a device address: the
// array's address on a device comes from hipGetSymbolAddress, looked up once per device (the first call on it,
// with that device current) and kept in scratch_ptr.
static __device__ __align__(256) unsigned char scratch[QB_GDN_STATIC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_ptr[kMaxDevices];
std::mutex scratch_mu;

// The current device's address of the scratch array.
std::string scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail("hipGetDevice", e);
  if (dev < 0 || dev >= kMaxDevices) return "gated delta: device index " + std::to_string(dev) + " out of range";
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) return hip_fail("hipGetSymbolAddress of the static scratch", e);
      scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return {};
}

// qb_gdn_bwd's body; with use_static the workspace is the current device's static scratch.
int bwd_impl(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g, const void* beta,
             const float* ckpt, const void* dy, const float* ds_out, void* dq, void* dk, void* dv, float* dg,
             void* dbeta, float* ds0, void* workspace, bool use_static, void* stream, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    Problem p{};
    std::string why = resolve(desc, p);
    const size_t el = p.in_bf16 ? 2 : 4, eo = p.out_bf16 ? 2 : 4;
    const bool any = p.BT > 0;
    const size_t need = why.empty() ? ws_bytes(desc, p) : 0;
    if (why.empty() && use_static && need > QB_GDN_STATIC_SCRATCH_BYTES)
      why = "gated delta: the backward without allocation needs " + std::to_string(need) +
            " bytes of scratch, more than its static " + std::to_string(size_t(QB_GDN_STATIC_SCRATCH_BYTES)) + " " +
            shape_of(*desc);
    const struct {
      const char* name;
      const void* ptr;
      bool req;
      size_t align;
    } ptrs[] = {{"q", q, any, 16},         {"k", k, any, 16},           {"v", v, any, el},
                {"g", g, any, 4},          {"beta", beta, any, el},     {"ckpt", ckpt, any, 16},
                {"dy", dy, any, eo},       {"ds_out", ds_out, false, 4}, {"dq", dq, any, eo},
                {"dk", dk, any, eo},       {"dv", dv, any, eo},         {"dg", dg, any, 4},
                {"dbeta", dbeta, any, eo}, {"ds0", ds0, false, 4},
                {"workspace", workspace, !use_static && why.empty() && any && need > 0, 16}};
    for (const auto& c : ptrs)
      if (why.empty()) why = check_ptr(c.name, c.ptr, c.req, c.align);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    if (use_static) {
      workspace = nullptr;
      if (any && need > 0) why = scratch_of_current_device(&workspace);
      if (!why.empty()) {
        set_err(err, errlen, why);
        return -1;
      }
    }
    const qbgdn::BwdPtrs a{q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0};
    hipStream_t s = static_cast<hipStream_t>(stream);
    qbgdn::Tracer tr = tracer_of(desc, s);
    const hipError_t e = desc->design == QB_GDN_RECURRENT ? qbgdn::rec_bwd(p, a, workspace, s, tr)
                                                          : qbgdn::chunk_bwd(p, a, workspace, s, tr);
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("backward launch", e));
      return -1;
    }
    return 0;
  });
}

}  // namespace

extern "C" {

int qb_gdn_bwd(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g,
               const void* beta, const float* ckpt, const void* dy, const float* ds_out, void* dq, void* dk, void* dv,
               float* dg, void* dbeta, float* ds0, void* workspace, void* stream, char* err, int errlen) {
  return bwd_impl(desc, q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0, workspace, false, stream, err,
                  errlen);
}

int qb_gdn_bwd_static(const qb_gdn_desc* desc, const void* q, const void* k, const void* v, const float* g,
                      const void* beta, const float* ckpt, const void* dy, const float* ds_out, void* dq, void* dk,
                      void* dv, float* dg, void* dbeta, float* ds0, void* stream, char* err, int errlen) {
  return bwd_impl(desc, q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0, nullptr, true, stream, err,
                  errlen);
}

}  // extern "C"

// ---- the pointwise neighbours ----------------------------------------------------------------------------------

namespace {

float round_bf16_host(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

// uses_dk / uses_dv: which of the widths the entry point runs on (the prologue Dk, the epilogue Dv).
std::string nb_resolve(const qb_gdn_desc* d, qbgdn::NbProblem& p, bool uses_dk, bool uses_dv) {
  if (!d) return "gated delta neighbours: null descriptor";
  const std::string sh = shape_of(*d);
  if (d->B < 1 || d->T < 0 || d->Hk < 1 || d->Hv < 1 || d->Dk < 1 || d->Dv < 1)
    return "gated delta neighbours: sizes must be positive " + sh;
  if (d->Hv % d->Hk) return "gated delta neighbours: value heads must be a multiple of key heads " + sh;
  if (d->dtype != QB_DTYPE_F32 && d->dtype != QB_DTYPE_BF16) return "gated delta neighbours: dtype must be f32 or bf16";
  const int64_t BT = int64_t(d->B) * d->T;
  if (BT * std::max(d->Hk * int64_t(d->Dk), d->Hv * int64_t(d->Dv)) > (int64_t(1) << 40))
    return "gated delta neighbours: problem too large " + sh;
  p = qbgdn::NbProblem{};
  p.BT = BT, p.Hk = d->Hk, p.Hv = d->Hv, p.Dk = d->Dk, p.Dv = d->Dv;
  p.bf16 = d->dtype == QB_DTYPE_BF16;
  // The reference's scalars: float(Dk^-1/2 * Dk^-1/2) and float(Dk^-1/2), in the activation dtype
  // (src/deltanet.cpp:95-97).
  const double inv = 1.0 / std::sqrt(double(d->Dk));
  p.scale_q = float(inv * inv), p.scale_k = float(inv);
  if (p.bf16) p.scale_q = round_bf16_host(p.scale_q), p.scale_k = round_bf16_host(p.scale_k);
  if (const char* why = qbgdn::nb_supports(p, uses_dk, uses_dv))
    return std::string("gated delta neighbours: ") + why + " " + sh;
  return {};
}

}  // namespace

extern "C" {

size_t qb_gdn_neighbours_workspace_bytes(const qb_gdn_desc* desc) {
  try {
    qbgdn::NbProblem p;
    if (!nb_resolve(desc, p, false, false).empty()) return 0;
    return qbgdn::nb_workspace_bytes(p);
  } catch (...) {
    return 0;
  }
}

int qb_gdn_prologue_fwd(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* a, const void* b,
                        const float* a_log, const float* dt_bias, void* q, void* k, void* beta, float* log_decay,
                        void* stream, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    qbgdn::NbProblem p;
    std::string why = nb_resolve(desc, p, true, false);
    const bool any = why.empty() && p.BT > 0;
    const size_t el = why.empty() && p.bf16 ? 2 : 4;
    const PtrCheck c[] = {{"q_raw", q_raw, any, 16}, {"k_raw", k_raw, any, 16}, {"a", a, any, el},
                          {"b", b, any, el},         {"a_log", a_log, true, 4},  {"dt_bias", dt_bias, true, 4},
                          {"q", q, any, 16},         {"k", k, any, 16},          {"beta", beta, any, el},
                          {"log_decay", log_decay, any, 4}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    const qbgdn::NbPrologue x{q_raw, k_raw, a, b, a_log, dt_bias, q, k, beta, log_decay};
    const hipError_t e = qbgdn::nb_prologue_fwd(p, x, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("prologue launch", e));
      return -1;
    }
    return 0;
  });
}

int qb_gdn_prologue_bwd(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* a, const void* b,
                        const float* a_log, const float* dt_bias, const void* dq, const void* dk, const void* dbeta,
                        const float* dlog_decay, void* dq_raw, void* dk_raw, void* da, void* db, float* da_log,
                        float* ddt_bias, void* workspace, void* stream, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    qbgdn::NbProblem p;
    std::string why = nb_resolve(desc, p, true, false);
    const bool any = why.empty() && p.BT > 0;
    const size_t el = why.empty() && p.bf16 ? 2 : 4;
    const PtrCheck c[] = {{"q_raw", q_raw, any, 16},   {"k_raw", k_raw, any, 16},     {"a", a, any, el},
                          {"b", b, any, el},           {"a_log", a_log, true, 4},      {"dt_bias", dt_bias, true, 4},
                          {"dq", dq, any, 16},         {"dk", dk, any, 16},            {"dbeta", dbeta, any, el},
                          {"dlog_decay", dlog_decay, any, 4}, {"dq_raw", dq_raw, any, 16}, {"dk_raw", dk_raw, any, 16},
                          {"da", da, any, el},         {"db", db, any, el},            {"da_log", da_log, true, 4},
                          {"ddt_bias", ddt_bias, true, 4},
                          {"workspace", workspace, why.empty() && qbgdn::nb_workspace_bytes(p) > 0, 4}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    const qbgdn::NbPrologueGrad x{q_raw, k_raw, a,  b,      a_log,  dt_bias, dq, dk,
                                  dbeta, dlog_decay, dq_raw, dk_raw, da, db, da_log, ddt_bias};
    const hipError_t e = qbgdn::nb_prologue_bwd(p, x, workspace, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("prologue backward launch", e));
      return -1;
    }
    return 0;
  });
}

int qb_gdn_fwd_prologue(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* v, const void* a,
                        const void* b, const float* a_log, const float* dt_bias, const float* s0, void* q, void* k,
                        void* beta, float* log_decay, void* y, float* s_out, float* ckpt, void* workspace,
                        void* stream, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    Problem p;
    std::string why = resolve(desc, p);
    qbgdn::NbProblem nb;
    if (why.empty()) why = nb_resolve(desc, nb, true, false);
    if (why.empty() && (desc->design != QB_GDN_CHUNKED || !desc->g_is_log || !p.in_bf16))
      why = "gated delta: the fused prologue runs the chunked design with bf16 inputs and g_is_log = 1 " +
            shape_of(*desc);
    const bool any = why.empty() && p.BT > 0;
    const size_t eo = p.out_bf16 ? 2 : 4;
    const PtrCheck c[] = {{"q_raw", q_raw, any, 16},      {"k_raw", k_raw, any, 16},     {"v", v, any, 2},
                          {"a", a, any, 2},               {"b", b, any, 2},              {"a_log", a_log, true, 4},
                          {"dt_bias", dt_bias, true, 4},  {"s0", s0, false, 4},          {"q", q, any, 16},
                          {"k", k, any, 16},              {"beta", beta, any, 2},        {"log_decay", log_decay, any, 4},
                          {"y", y, any, eo},              {"s_out", s_out, false, 4},    {"ckpt", ckpt, false, 16},
                          {"workspace", workspace, any && ws_bytes(desc, p) > 0, 16}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    const qbgdn::PrologueIn pro{q_raw, k_raw, a, b, a_log, dt_bias, nb.scale_q, nb.scale_k, q, k, beta, log_decay};
    const qbgdn::FwdPtrs f{q, k, v, log_decay, beta, s0, y, s_out, ckpt};
    hipStream_t st = static_cast<hipStream_t>(stream);
    qbgdn::Tracer tr = tracer_of(desc, st);
    const hipError_t e = qbgdn::chunk_fwd_prologue(p, pro, f, workspace, st, tr);
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("forward launch", e));
      return -1;
    }
    return 0;
  });
}

int qb_gdn_bwd_prologue(const qb_gdn_desc* desc, const void* q_raw, const void* k_raw, const void* a, const void* b,
                        const float* a_log, const float* dt_bias, const void* q, const void* k, const void* v,
                        const void* beta, const float* log_decay, const float* ckpt, const void* dy,
                        const float* ds_out, void* dq_raw, void* dk_raw, void* dv, void* da, void* db, float* da_log,
                        float* ddt_bias, float* ds0, void* workspace, void* stream, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    Problem p;
    std::string why = resolve(desc, p);
    qbgdn::NbProblem nb;
    if (why.empty()) why = nb_resolve(desc, nb, true, false);
    if (why.empty() && (desc->design != QB_GDN_CHUNKED || !desc->g_is_log || !p.in_bf16 || !p.out_bf16))
      why = "gated delta: the fused prologue backward runs the chunked design with bf16 inputs and outputs and "
            "g_is_log = 1 " + shape_of(*desc);
    const bool any = why.empty() && p.BT > 0;
    const PtrCheck c[] = {{"q_raw", q_raw, any, 16},         {"k_raw", k_raw, any, 16},
                          {"a", a, any, 2},                  {"b", b, any, 2},
                          {"a_log", a_log, true, 4},         {"dt_bias", dt_bias, true, 4},
                          {"q", q, any, 16},                 {"k", k, any, 16},
                          {"v", v, any, 2},                  {"beta", beta, any, 2},
                          {"log_decay", log_decay, any, 4},  {"ckpt", ckpt, any, 16},
                          {"dy", dy, any, 2},                {"ds_out", ds_out, false, 4},
                          {"dq_raw", dq_raw, any, 16},       {"dk_raw", dk_raw, any, 16},
                          {"dv", dv, any, 2},                {"da", da, any, 2},
                          {"db", db, any, 2},                {"da_log", da_log, true, 4},
                          {"ddt_bias", ddt_bias, true, 4},   {"ds0", ds0, false, 4},
                          {"workspace", workspace, any && ws_bytes(desc, p) > 0, 16}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const qbgdn::PrologueGradIn pro{q_raw, k_raw, a, b, a_log, dt_bias, nb.scale_q, nb.scale_k,
                                    dq_raw, dk_raw, da, db, da_log, ddt_bias};
    const qbgdn::BwdPtrs bp{q, k, v, log_decay, beta, ckpt, dy, ds_out, dq_raw, dk_raw, dv, nullptr, nullptr, ds0};
    qbgdn::Tracer tr = tracer_of(desc, st);
    const hipError_t e = qbgdn::chunk_bwd_prologue(p, pro, bp, workspace, st, tr);
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("backward launch", e));
      return -1;
    }
    return 0;
  });
}

int qb_gdn_epilogue_fwd(const qb_gdn_desc* desc, const void* y, const void* z, const float* norm_w, float eps, void* o,
                        void* stream, char* err, int errlen) {
  return guarded(err, errlen, [&] {
    qbgdn::NbProblem p;
    std::string why = nb_resolve(desc, p, false, true);
    if (why.empty() && !(eps > 0.f)) why = "gated delta neighbours: eps must be positive";
    const bool any = why.empty() && p.BT > 0;
    const PtrCheck c[] = {{"y", y, any, 16}, {"z", z, any, 16}, {"norm_w", norm_w, true, 16}, {"o", o, any, 16}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    const qbgdn::NbEpilogue x{y, z, norm_w, eps, o};
    const hipError_t e = qbgdn::nb_epilogue_fwd(p, x, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("epilogue launch", e));
      return -1;
    }
    return 0;
  });
}

int qb_gdn_epilogue_bwd(const qb_gdn_desc* desc, const void* y, const void* z, const float* norm_w, float eps,
                        const void* dout, void* dy, void* dz, float* dnorm_w, void* workspace, void* stream, char* err,
                        int errlen) {
  return guarded(err, errlen, [&] {
    qbgdn::NbProblem p;
    std::string why = nb_resolve(desc, p, false, true);
    if (why.empty() && !(eps > 0.f)) why = "gated delta neighbours: eps must be positive";
    const bool any = why.empty() && p.BT > 0;
    const PtrCheck c[] = {{"y", y, any, 16},       {"z", z, any, 16},   {"norm_w", norm_w, true, 16},
                          {"dout", dout, any, 16}, {"dy", dy, any, 16}, {"dz", dz, any, 16},
                          {"dnorm_w", dnorm_w, true, 4},
                          {"workspace", workspace, why.empty() && qbgdn::nb_workspace_bytes(p) > 0, 4}};
    if (why.empty()) why = check_all(c);
    if (!why.empty()) {
      set_err(err, errlen, why);
      return -1;
    }
    const qbgdn::NbEpilogueGrad x{y, z, norm_w, eps, dout, dy, dz, dnorm_w};
    const hipError_t e = qbgdn::nb_epilogue_bwd(p, x, workspace, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      set_err(err, errlen, hip_fail("epilogue backward launch", e));
      return -1;
    }
    return 0;
  });
}

}  // extern "C"
