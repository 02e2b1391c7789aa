// The C++ adapters of include/qb: qb::array and the reference's entry points gated_delta (src/deltanet.cpp:49-61),
// gated_delta_trainable and gated_delta_vjp (src/delta_grad.cpp:155-212) on top of the C ABI of qb_gdn.h.
// A failed ABI call (-1 and a message) becomes std::runtime_error with that message, as the reference throws.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>
#include <string>

#include "gdn_common.h"
#include "qb/delta_grad.h"
#include "qb/deltanet.h"
#include "qb/neighbours.h"
#include "qb_gdn.h"

namespace qb {
namespace {

void* g_stream = nullptr;

hipStream_t cur() { return static_cast<hipStream_t>(g_stream); }

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string("gated delta: ") + what + ": " + hipGetErrorString(e));
}

void* device_alloc(size_t bytes) {
  void* p = nullptr;
  if (bytes) check(hipMalloc(&p, bytes), "hipMalloc");
  return p;
}

std::string shape_str(const Shape& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

__global__ void cast_kernel(const void* src, void* dst, int64_t n, int to_bf16) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (to_bf16)
    static_cast<qbgdn::bf16_t*>(dst)[i] = qbgdn::f32_to_bf16(static_cast<const float*>(src)[i]);
  else
    static_cast<float*>(dst)[i] = qbgdn::bf16_to_f32(static_cast<const qbgdn::bf16_t*>(src)[i]);
}

// A fill kernel rather than hipMemsetAsync, which must not be recorded into graphs a caller may capture.
__global__ void zero_kernel(uint32_t* dst, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = 0u;
}

// Scratch device memory for one call, released in stream order.
struct Scratch {
  void* p = nullptr;
  explicit Scratch(size_t bytes) {
    if (bytes) check(hipMallocAsync(&p, bytes, cur()), "hipMallocAsync");
  }
  ~Scratch() {
    if (p) (void)hipFreeAsync(p, cur());
  }
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
};

// The design the adapters run: the chunked one where the library supports the shape and T > 40, else the recurrent
// one, which is the faster up to a few dozen steps (4B layer shape, launches included: forward + backward 43.7
// against 47.0 us at T = 32, 53.0 against 47.4 us at T = 48, the two crossing near T = 38; a one-token decode call
// about 6 us against 15 us).
int pick_design(qb_gdn_desc d) {
  char err[16];
  if (d.T <= 40) return QB_GDN_RECURRENT;
  d.design = QB_GDN_CHUNKED;
  if (qb_gdn_validate(&d, err, sizeof err) == 0) return QB_GDN_CHUNKED;
  return QB_GDN_RECURRENT;
}

// Shapes of one call, checked against each other; the messages name every shape, as the reference's do.
struct Problem {
  int B, T, Hk, Dk, Hv, Dv;
};

Problem check_shapes(const char* who, const array& q, const array& k, const array& v, const array& g,
                     const array& beta, const array& state) {
  auto fail = [&](const std::string& why) {
    throw std::runtime_error(std::string(who) + ": " + why + " (q " + shape_str(q.shape()) + ", k " +
                             shape_str(k.shape()) + ", v " + shape_str(v.shape()) + ", g " + shape_str(g.shape()) +
                             ", beta " + shape_str(beta.shape()) + ", state " + shape_str(state.shape()) + ")");
  };
  if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4 || g.ndim() != 3 || beta.ndim() != 3 || state.ndim() != 4)
    fail("q, k, v, state need 4 dimensions and g, beta 3");
  const Problem p{q.shape(0), q.shape(1), q.shape(2), q.shape(3), v.shape(2), v.shape(3)};
  if (k.shape() != q.shape()) fail("k must have q's shape");
  if (v.shape(0) != p.B || v.shape(1) != p.T) fail("v must match q in batch and time");
  const Shape bth{p.B, p.T, p.Hv};
  if (g.shape() != bth || beta.shape() != bth) fail("g and beta must be [B, T, Hv]");
  if (state.shape() != Shape{p.B, p.Hv, p.Dv, p.Dk}) fail("state must be [B, Hv, Dv, Dk]");
  return p;
}

qb_gdn_desc make_desc(const Problem& p, Dtype io, bool out_f32) {
  qb_gdn_desc d{};
  d.B = p.B, d.T = p.T, d.Hk = p.Hk, d.Hv = p.Hv, d.Dk = p.Dk, d.Dv = p.Dv;
  d.chunk = 64;
  d.dtype = int(io);
  d.g_is_log = 0;  // the reference's decay factor; the library takes logs and returns dL/dg
  d.out_f32 = out_f32 ? 1 : 0;
  d.design = pick_design(d);
  return d;
}

// The ABI's element type for q, k, v, beta: bfloat16 when all four are, else float32 (the reference computes in
// float32 whatever it is fed, src/deltanet.cpp:54).
Dtype io_dtype(const array& q, const array& k, const array& v, const array& beta) {
  const bool bf = q.dtype() == bfloat16 && k.dtype() == bfloat16 && v.dtype() == bfloat16 &&
                  beta.dtype() == bfloat16;
  return bf ? bfloat16 : float32;
}

// Forward through the ABI; ckpt may be null.
void run_fwd(const qb_gdn_desc& d, const array& q, const array& k, const array& v, const array& g,
             const array& beta, const array& s0, array& y, array& s_out, float* ckpt) {
  Scratch ws(qb_gdn_workspace_bytes(&d));
  char err[512];
  if (qb_gdn_fwd(&d, q.data(), k.data(), v.data(), static_cast<const float*>(g.data()), beta.data(),
                 static_cast<const float*>(s0.data()), y.data(), static_cast<float*>(s_out.data()), ckpt, ws.p,
                 g_stream, err, sizeof err) != 0)
    throw std::runtime_error(err);
}

// The neighbours' descriptor: B, T, heads and widths, the activations' dtype (the other fields are unused).
qb_gdn_desc nb_desc(int B, int T, int Hk, int Hv, int Dk, int Dv, Dtype act) {
  qb_gdn_desc d{};
  d.B = B, d.T = T, d.Hk = Hk, d.Hv = Hv, d.Dk = Dk, d.Dv = Dv;
  d.chunk = 64;
  d.dtype = int(act);
  return d;
}

Dtype act_dtype(std::initializer_list<const array*> xs) {
  for (const array* x : xs)
    if (x->dtype() != bfloat16) return float32;
  return bfloat16;
}

void need(bool ok, const char* who, const std::string& why, std::initializer_list<const array*> xs) {
  if (ok) return;
  std::string m = std::string(who) + ": " + why + " (shapes";
  for (const array* x : xs) m += " " + shape_str(x->shape());
  throw std::runtime_error(m + ")");
}

void abi(int rc, const char* err) {
  if (rc != 0) throw std::runtime_error(err);
}

const float* fp(const array& x) { return static_cast<const float*>(x.data()); }
float* fp(array& x) { return static_cast<float*>(x.data()); }

// The shapes of the prologue fused into the recurrence, checked against each other.
Problem check_fused(const char* who, const array& q_raw, const array& k_raw, const array& v, const array& a,
                    const array& b, const array& a_log, const array& dt_bias, const array& state) {
  need(q_raw.ndim() == 4 && k_raw.shape() == q_raw.shape() && v.ndim() == 4 && a.ndim() == 3 && b.shape() == a.shape(),
       who, "q_raw, k_raw must be [B, T, Hk, Dk], v [B, T, Hv, Dv] and a, b [B, T, Hv]", {&q_raw, &k_raw, &v, &a, &b});
  const Problem p{q_raw.shape(0), q_raw.shape(1), q_raw.shape(2), q_raw.shape(3), v.shape(2), v.shape(3)};
  need(v.shape(0) == p.B && v.shape(1) == p.T && a.shape() == Shape{p.B, p.T, p.Hv}, who,
       "v, a, b must match q_raw in batch and time, with v's Hv heads", {&q_raw, &v, &a});
  need(a_log.shape() == Shape{p.Hv} && dt_bias.shape() == Shape{p.Hv}, who, "a_log and dt_bias must be [Hv]",
       {&a, &a_log, &dt_bias});
  need(state.empty() || state.shape() == Shape{p.B, p.Hv, p.Dv, p.Dk}, who, "state must be [B, Hv, Dv, Dk] or empty",
       {&v, &state});
  need(act_dtype({&q_raw, &k_raw, &v, &a, &b}) == bfloat16, who, "the fused prologue takes bfloat16 activations",
       {&q_raw, &v, &a});
  return p;
}

qb_gdn_desc fused_desc(const Problem& p) {
  qb_gdn_desc d = make_desc(p, bfloat16, false);
  d.g_is_log = 1;  // the prologue emits the log-decay
  d.design = QB_GDN_CHUNKED;
  return d;
}

}  // namespace

size_t size_of(Dtype dtype) { return dtype == bfloat16 ? 2 : 4; }

array::array(Shape shape, Dtype dtype) : shape_(std::move(shape)), dtype_(dtype) {
  for (int s : shape_)
    if (s < 0) throw std::runtime_error("qb::array: negative dimension in " + shape_str(shape_));
  buf_ = std::shared_ptr<void>(device_alloc(std::max<size_t>((nbytes() + 3) / 4 * 4, 4)),
                               [](void* p) { (void)hipFree(p); });
}

array array::from_host(const void* data, Shape shape, Dtype dtype) {
  array a(std::move(shape), dtype);
  check(hipMemcpyAsync(a.data(), data, a.nbytes(), hipMemcpyHostToDevice, cur()), "hipMemcpyAsync");
  check(hipStreamSynchronize(cur()), "hipStreamSynchronize");
  return a;
}

array array::zeros(Shape shape, Dtype dtype) {
  array a(std::move(shape), dtype);
  const int64_t words = int64_t((a.nbytes() + 3) / 4);  // the buffer is at least 4-byte aligned and padded
  if (words) {
    hipLaunchKernelGGL(zero_kernel, dim3(unsigned((words + 255) / 256)), dim3(256), 0, cur(),
                       static_cast<uint32_t*>(a.data()), words);
    check(hipGetLastError(), "zero kernel");
  }
  return a;
}

void array::to_host(void* dst) const {
  check(hipMemcpyAsync(dst, data(), nbytes(), hipMemcpyDeviceToHost, cur()), "hipMemcpyAsync");
  check(hipStreamSynchronize(cur()), "hipStreamSynchronize");
}

int array::shape(int dim) const {
  const int n = ndim();
  if (dim < -n || dim >= n) throw std::runtime_error("qb::array: dimension " + std::to_string(dim) + " of " +
                                                     shape_str(shape_));
  return shape_[dim < 0 ? dim + n : dim];
}

size_t array::size() const {
  size_t n = 1;
  for (int s : shape_) n *= size_t(s);
  return n;
}

array astype(const array& x, Dtype dtype) {
  if (x.dtype() == dtype) return x;
  array r(x.shape(), dtype);
  const int64_t n = int64_t(x.size());
  if (n) {
    hipLaunchKernelGGL(cast_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, cur(), x.data(), r.data(), n,
                       dtype == bfloat16 ? 1 : 0);
    check(hipGetLastError(), "cast kernel");
  }
  return r;
}

void set_stream(void* s) { g_stream = s; }
void* stream() { return g_stream; }

std::pair<array, array> gated_delta_trainable(const array& q, const array& k, const array& v, const array& g,
                                              const array& beta, const array& state) {
  const Problem p = check_shapes("gated delta", q, k, v, g, beta, state);
  const Dtype io = io_dtype(q, k, v, beta);
  const qb_gdn_desc d = make_desc(p, io, false);
  array y({p.B, p.T, p.Hv, p.Dv}, io), s_out({p.B, p.Hv, p.Dv, p.Dk}, float32);
  run_fwd(d, astype(q, io), astype(k, io), astype(v, io), astype(g, float32), astype(beta, io),
          astype(state, float32), y, s_out, nullptr);
  return {y, s_out};
}

std::pair<array, array> gated_delta(const array& q, const array& k, const array& v, const array& g,
                                    const array& beta, const array& state, bool train) {
  // The trainable op's forward is the same computation (src/deltanet.cpp:55-60); y returns in q's dtype.
  (void)train;
  auto [y, s] = gated_delta_trainable(q, k, v, g, beta, state);
  return {astype(y, q.dtype()), s};
}

std::vector<array> gated_delta_vjp(const std::vector<array>& in, const array& dy, const array& dstate) {
  if (in.size() != 6)
    throw std::runtime_error("gated delta backward: needs 6 primals (q, k, v, g, beta, state), got " +
                             std::to_string(in.size()));
  const array &q = in[0], &k = in[1], &v = in[2], &g = in[3], &beta = in[4], &state = in[5];
  const Problem p = check_shapes("gated delta backward", q, k, v, g, beta, state);
  if (dy.shape() != Shape{p.B, p.T, p.Hv, p.Dv})
    throw std::runtime_error("gated delta backward: dy must be " + shape_str({p.B, p.T, p.Hv, p.Dv}) + ", got " +
                             shape_str(dy.shape()));
  if (!dstate.empty() && dstate.shape() != state.shape())
    throw std::runtime_error("gated delta backward: dstate must be " + shape_str(state.shape()) + ", got " +
                             shape_str(dstate.shape()));
  const Dtype io = io_dtype(q, k, v, beta);
  // Cotangents in float32 unless every tensor of the output side is bfloat16.
  const bool out_f32 = io == float32 || dy.dtype() == float32;
  const Dtype od = out_f32 ? float32 : bfloat16;
  const qb_gdn_desc d = make_desc(p, io, out_f32);
  const array qi = astype(q, io), ki = astype(k, io), vi = astype(v, io), bi = astype(beta, io);
  const array gi = astype(g, float32), s0 = astype(state, float32);

  // The chunk-start states from the forward itself (the reference rebuilds them, src/delta_grad.cpp:172-181).
  Scratch ckpt(qb_gdn_ckpt_bytes(&d));
  {
    array y({p.B, p.T, p.Hv, p.Dv}, od), s_out({p.B, p.Hv, p.Dv, p.Dk}, float32);
    run_fwd(d, qi, ki, vi, gi, bi, s0, y, s_out, static_cast<float*>(ckpt.p));
  }
  const array dyi = astype(dy, od);
  const array dsi = dstate.empty() ? array() : astype(dstate, float32);
  array dq({p.B, p.T, p.Hk, p.Dk}, od), dk({p.B, p.T, p.Hk, p.Dk}, od), dv({p.B, p.T, p.Hv, p.Dv}, od);
  array dg({p.B, p.T, p.Hv}, float32), db({p.B, p.T, p.Hv}, od), ds0({p.B, p.Hv, p.Dv, p.Dk}, float32);
  Scratch ws(qb_gdn_workspace_bytes(&d));
  char err[512];
  if (qb_gdn_bwd(&d, qi.data(), ki.data(), vi.data(), static_cast<const float*>(gi.data()), bi.data(),
                 static_cast<const float*>(ckpt.p), dyi.data(), static_cast<const float*>(dsi.data()), dq.data(),
                 dk.data(), dv.data(), static_cast<float*>(dg.data()), db.data(), static_cast<float*>(ds0.data()),
                 ws.p, g_stream, err, sizeof err) != 0)
    throw std::runtime_error(err);
  return {astype(dq, q.dtype()), astype(dk, k.dtype()),  astype(dv, v.dtype()),
          astype(dg, g.dtype()), astype(db, beta.dtype()), astype(ds0, state.dtype())};
}

Prologue deltanet_prologue(const array& q_raw, const array& k_raw, const array& a, const array& b,
                           const array& a_log, const array& dt_bias) {
  const char* who = "deltanet prologue";
  need(q_raw.ndim() == 4 && k_raw.shape() == q_raw.shape() && a.ndim() == 3 && b.shape() == a.shape(), who,
       "q_raw, k_raw must be [B, T, Hk, Dk] and a, b [B, T, Hv]", {&q_raw, &k_raw, &a, &b});
  const int B = q_raw.shape(0), T = q_raw.shape(1), Hk = q_raw.shape(2), Dk = q_raw.shape(3), Hv = a.shape(2);
  need(a.shape(0) == B && a.shape(1) == T && a_log.shape() == Shape{Hv} && dt_bias.shape() == Shape{Hv}, who,
       "a, b must match q_raw in batch and time, and a_log, dt_bias be [Hv]", {&q_raw, &a, &a_log, &dt_bias});
  const Dtype act = act_dtype({&q_raw, &k_raw, &a, &b});
  const qb_gdn_desc d = nb_desc(B, T, Hk, Hv, Dk, Dk, act);
  const array qr = astype(q_raw, act), kr = astype(k_raw, act), aa = astype(a, act), bb = astype(b, act);
  const array al = astype(a_log, float32), dt = astype(dt_bias, float32);
  Prologue r{array(q_raw.shape(), act), array(q_raw.shape(), act), array(a.shape(), act), array(a.shape(), float32)};
  char err[512];
  abi(qb_gdn_prologue_fwd(&d, qr.data(), kr.data(), aa.data(), bb.data(), fp(al), fp(dt), r.q.data(), r.k.data(),
                          r.beta.data(), fp(r.log_decay), g_stream, err, sizeof err),
      err);
  return r;
}

PrologueGrads deltanet_prologue_vjp(const array& q_raw, const array& k_raw, const array& a, const array& b,
                                    const array& a_log, const array& dt_bias, const array& dq, const array& dk,
                                    const array& dbeta, const array& dlog_decay) {
  const char* who = "deltanet prologue backward";
  need(q_raw.ndim() == 4 && k_raw.shape() == q_raw.shape() && dq.shape() == q_raw.shape() &&
           dk.shape() == q_raw.shape() && a.ndim() == 3 && b.shape() == a.shape() && dbeta.shape() == a.shape() &&
           dlog_decay.shape() == a.shape(),
       who, "cotangents must have their primals' shapes", {&q_raw, &k_raw, &a, &b, &dq, &dk, &dbeta, &dlog_decay});
  const int B = q_raw.shape(0), T = q_raw.shape(1), Hk = q_raw.shape(2), Dk = q_raw.shape(3), Hv = a.shape(2);
  need(a.shape(0) == B && a.shape(1) == T && a_log.shape() == Shape{Hv} && dt_bias.shape() == Shape{Hv}, who,
       "a, b must match q_raw in batch and time, and a_log, dt_bias be [Hv]", {&q_raw, &a, &a_log, &dt_bias});
  const Dtype act = act_dtype({&q_raw, &k_raw, &a, &b});
  const qb_gdn_desc d = nb_desc(B, T, Hk, Hv, Dk, Dk, act);
  const array qr = astype(q_raw, act), kr = astype(k_raw, act), aa = astype(a, act), bb = astype(b, act);
  const array al = astype(a_log, float32), dt = astype(dt_bias, float32);
  const array gq = astype(dq, act), gk = astype(dk, act), gb = astype(dbeta, act), gl = astype(dlog_decay, float32);
  PrologueGrads r{array(q_raw.shape(), act), array(q_raw.shape(), act), array(a.shape(), act),
                  array(a.shape(), act),     array({Hv}, float32),      array({Hv}, float32)};
  Scratch ws(qb_gdn_neighbours_workspace_bytes(&d));
  char err[512];
  abi(qb_gdn_prologue_bwd(&d, qr.data(), kr.data(), aa.data(), bb.data(), fp(al), fp(dt), gq.data(), gk.data(),
                          gb.data(), fp(gl), r.dq_raw.data(), r.dk_raw.data(), r.da.data(), r.db.data(),
                          fp(r.da_log), fp(r.ddt_bias), ws.p, g_stream, err, sizeof err),
      err);
  return r;
}

array deltanet_epilogue(const array& y, const array& z, const array& norm_w, float eps) {
  const char* who = "deltanet epilogue";
  need(y.ndim() == 4 && z.shape() == y.shape() && norm_w.shape() == Shape{y.shape(3)}, who,
       "y, z must be [B, T, Hv, Dv] and norm_w [Dv]", {&y, &z, &norm_w});
  const Dtype act = act_dtype({&y, &z});
  const int Hv = y.shape(2), Dv = y.shape(3);
  const qb_gdn_desc d = nb_desc(y.shape(0), y.shape(1), Hv, Hv, Dv, Dv, act);
  const array yy = astype(y, act), zz = astype(z, act), w = astype(norm_w, float32);
  array o(y.shape(), act);
  char err[512];
  abi(qb_gdn_epilogue_fwd(&d, yy.data(), zz.data(), fp(w), eps, o.data(), g_stream, err, sizeof err), err);
  return o;
}

EpilogueGrads deltanet_epilogue_vjp(const array& y, const array& z, const array& norm_w, float eps,
                                    const array& dout) {
  const char* who = "deltanet epilogue backward";
  need(y.ndim() == 4 && z.shape() == y.shape() && dout.shape() == y.shape() && norm_w.shape() == Shape{y.shape(3)},
       who, "y, z, dout must be [B, T, Hv, Dv] and norm_w [Dv]", {&y, &z, &dout, &norm_w});
  const Dtype act = act_dtype({&y, &z});
  const int Hv = y.shape(2), Dv = y.shape(3);
  const qb_gdn_desc d = nb_desc(y.shape(0), y.shape(1), Hv, Hv, Dv, Dv, act);
  const array yy = astype(y, act), zz = astype(z, act), w = astype(norm_w, float32), go = astype(dout, act);
  EpilogueGrads r{array(y.shape(), act), array(y.shape(), act), array({Dv}, float32)};
  Scratch ws(qb_gdn_neighbours_workspace_bytes(&d));
  char err[512];
  abi(qb_gdn_epilogue_bwd(&d, yy.data(), zz.data(), fp(w), eps, go.data(), r.dy.data(), r.dz.data(), fp(r.dnorm_w),
                          ws.p, g_stream, err, sizeof err),
      err);
  return r;
}

PrologueRecurrence deltanet_prologue_recurrence(const array& q_raw, const array& k_raw, const array& v,
                                                const array& a, const array& b, const array& a_log,
                                                const array& dt_bias, const array& state) {
  const Problem p = check_fused("deltanet prologue + recurrence", q_raw, k_raw, v, a, b, a_log, dt_bias, state);
  const qb_gdn_desc d = fused_desc(p);
  const array al = astype(a_log, float32), dt = astype(dt_bias, float32);
  const array s0 = state.empty() ? array() : astype(state, float32);
  PrologueRecurrence r{array(v.shape(), bfloat16),     array({p.B, p.Hv, p.Dv, p.Dk}, float32),
                       array(q_raw.shape(), bfloat16), array(k_raw.shape(), bfloat16),
                       array(a.shape(), bfloat16),     array(a.shape(), float32)};
  Scratch ws(qb_gdn_workspace_bytes(&d));
  char err[512];
  abi(qb_gdn_fwd_prologue(&d, q_raw.data(), k_raw.data(), v.data(), a.data(), b.data(), fp(al), fp(dt), fp(s0),
                          r.q.data(), r.k.data(), r.beta.data(), fp(r.log_decay), r.y.data(), fp(r.state), nullptr,
                          ws.p, g_stream, err, sizeof err),
      err);
  return r;
}

PrologueRecurrenceGrads deltanet_prologue_recurrence_vjp(const array& q_raw, const array& k_raw, const array& v,
                                                         const array& a, const array& b, const array& a_log,
                                                         const array& dt_bias, const array& state, const array& dy,
                                                         const array& dstate) {
  const char* who = "deltanet prologue + recurrence backward";
  const Problem p = check_fused(who, q_raw, k_raw, v, a, b, a_log, dt_bias, state);
  need(dy.shape() == v.shape(), who, "dy must have v's shape", {&v, &dy});
  need(dstate.empty() || dstate.shape() == Shape{p.B, p.Hv, p.Dv, p.Dk}, who,
       "dstate must be [B, Hv, Dv, Dk] or empty", {&v, &dstate});
  const qb_gdn_desc d = fused_desc(p);
  const array al = astype(a_log, float32), dt = astype(dt_bias, float32);
  const array s0 = state.empty() ? array() : astype(state, float32);
  // The forward again, keeping the chunk-start states and the recurrence's inputs (as gated_delta_vjp rebuilds the
  // states, src/delta_grad.cpp:172-181).
  Scratch ckpt(qb_gdn_ckpt_bytes(&d));
  array q(q_raw.shape(), bfloat16), k(k_raw.shape(), bfloat16), beta(a.shape(), bfloat16), ld(a.shape(), float32);
  char err[512];
  {
    array y(v.shape(), bfloat16), s_out({p.B, p.Hv, p.Dv, p.Dk}, float32);
    Scratch ws(qb_gdn_workspace_bytes(&d));
    abi(qb_gdn_fwd_prologue(&d, q_raw.data(), k_raw.data(), v.data(), a.data(), b.data(), fp(al), fp(dt), fp(s0),
                            q.data(), k.data(), beta.data(), fp(ld), y.data(), fp(s_out),
                            static_cast<float*>(ckpt.p), ws.p, g_stream, err, sizeof err),
        err);
  }
  const array dyi = astype(dy, bfloat16);
  const array dsi = dstate.empty() ? array() : astype(dstate, float32);
  PrologueRecurrenceGrads r{array(q_raw.shape(), bfloat16), array(k_raw.shape(), bfloat16),
                            array(v.shape(), bfloat16),     array(a.shape(), bfloat16),
                            array(b.shape(), bfloat16),     array({p.Hv}, float32),
                            array({p.Hv}, float32),         array({p.B, p.Hv, p.Dv, p.Dk}, float32)};
  Scratch ws(qb_gdn_workspace_bytes(&d));
  abi(qb_gdn_bwd_prologue(&d, q_raw.data(), k_raw.data(), a.data(), b.data(), fp(al), fp(dt), q.data(), k.data(),
                          v.data(), beta.data(), fp(ld), static_cast<const float*>(ckpt.p), dyi.data(), fp(dsi),
                          r.dq_raw.data(), r.dk_raw.data(), r.dv.data(), r.da.data(), r.db.data(), fp(r.da_log),
                          fp(r.ddt_bias), fp(r.dstate), ws.p, g_stream, err, sizeof err),
      err);
  return r;
}

std::pair<array, array> gated_delta_rows(const array& q, const array& k, const array& v, const array& g,
                                         const array& beta, const array& state) {
  const Problem p = check_shapes("gated delta rows", q, k, v, g, beta, state);
  const Dtype io = io_dtype(q, k, v, beta);
  qb_gdn_desc d = make_desc(p, io, false);
  d.design = QB_GDN_RECURRENT;
  array y({p.B, p.T, p.Hv, p.Dv}, io), rows({p.B, p.T, p.Hv, p.Dv, p.Dk}, float32);
  const array qq = astype(q, io), kk = astype(k, io), vv = astype(v, io), gg = astype(g, float32);
  const array bb = astype(beta, io), s0 = astype(state, float32);
  char err[512];
  abi(qb_gdn_fwd_rows(&d, qq.data(), kk.data(), vv.data(), fp(gg), bb.data(), fp(s0), y.data(), fp(rows), g_stream,
                      err, sizeof err),
      err);
  return {astype(y, q.dtype()), rows};
}

}  // namespace qb
