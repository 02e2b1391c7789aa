// Checks the C++ adapters of include/qb (gated_delta, gated_delta_trainable, gated_delta_vjp, gated_delta_rows)
// against the oracle, the neighbours' adapters (deltanet_prologue / _epilogue and their vjps) in float32
// against a float64 statement of their formulas here, and the prologue fused into the recurrence
// (deltanet_prologue_recurrence and its vjp) against the separate steps it replaces, bit for bit,
// the way the reference's tests check its entry points (tests/test_deltanet.cpp:25-154): seeded inputs, the
// forward and every cotangent compared normwise, max|X - X_ref| / max|X_ref|. float32 outputs must be within 2e-3;
// a bfloat16 output may in addition differ by half a bfloat16 ulp of each reference element (its own rounding).
// Also checks that bad shapes throw std::runtime_error naming them. Prints PASS and exits 0, or FAIL and exits 1.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../oracle/gdn_ref.h"
#include "qb_gdn.h"
#include "qb/delta_grad.h"
#include "qb/deltanet.h"
#include "qb/neighbours.h"

namespace {

int failures = 0;

uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
float from_bf16(uint16_t b) {
  const uint32_t u = uint32_t(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

struct Rng {  // splitmix64 and Box-Muller
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  double uniform() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
  float normal() {
    const double u = uniform() + 1e-300, v = uniform();
    return float(std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v));
  }
};

// Host values (already representable in dtype) and their device array.
struct Tensor {
  std::vector<float> host;
  qb::array dev;
};

Tensor make(std::vector<float> x, qb::Shape shape, qb::Dtype dt) {
  if (dt == qb::bfloat16) {
    std::vector<uint16_t> b(x.size());
    for (size_t i = 0; i < x.size(); ++i) b[i] = to_bf16(x[i]), x[i] = from_bf16(b[i]);
    return {x, qb::array::from_host(b.data(), shape, dt)};
  }
  return {x, qb::array::from_host(x.data(), shape, dt)};
}

std::vector<float> fetch(const qb::array& a) {
  std::vector<float> r(a.size());
  if (a.dtype() == qb::bfloat16) {
    std::vector<uint16_t> b(a.size());
    a.to_host(b.data());
    for (size_t i = 0; i < b.size(); ++i) r[i] = from_bf16(b[i]);
  } else {
    a.to_host(r.data());
  }
  return r;
}

void compare(const char* what, const qb::array& got_dev, const std::vector<float>& ref, double tol) {
  const std::vector<float> got = fetch(got_dev);
  const bool bf = got_dev.dtype() == qb::bfloat16;
  double mref = 0, merr = 0;
  for (size_t i = 0; i < ref.size(); ++i) mref = std::fmax(mref, std::fabs(ref[i]));
  for (size_t i = 0; i < ref.size(); ++i) {
    double e = std::fabs(double(got[i]) - ref[i]);
    if (bf && ref[i] != 0.f) {  // half a bfloat16 ulp of the reference element
      int ex;
      std::frexp(ref[i], &ex);
      e = std::fmax(0.0, e - std::ldexp(1.0, ex - 9));
    }
    merr = std::fmax(merr, e);
  }
  const double rel = mref > 0 ? merr / mref : merr;
  const bool ok = got.size() == ref.size() && rel <= tol;
  std::printf("  %-6s %s normwise %.3e (tol %.0e)%s\n", what, bf ? "bf16" : "f32 ", rel, tol, ok ? "" : "  <-- FAIL");
  failures += !ok;
}

void run_case(const char* name, int B, int T, int Hk, int Hv, int Dk, int Dv, qb::Dtype dt, uint64_t seed) {
  std::printf("case %s: B=%d T=%d Hk=%d Hv=%d Dk=%d Dv=%d %s\n", name, B, T, Hk, Hv, Dk, Dv,
              dt == qb::bfloat16 ? "bf16" : "f32");
  Rng r{seed};
  const size_t nqk = size_t(B) * T * Hk * Dk, nv = size_t(B) * T * Hv * Dv, ng = size_t(B) * T * Hv;
  const size_t ns = size_t(B) * Hv * Dv * Dk;
  std::vector<float> q(nqk), k(nqk), v(nv), g(ng), beta(ng), s0(ns), dy(nv), ds(ns);
  for (auto* x : {&q, &k})
    for (size_t row = 0; row < nqk / Dk; ++row) {  // unit norm over Dk
      double n = 0;
      for (int c = 0; c < Dk; ++c) (*x)[row * Dk + c] = r.normal(), n += double((*x)[row * Dk + c]) * (*x)[row * Dk + c];
      for (int c = 0; c < Dk; ++c) (*x)[row * Dk + c] = float((*x)[row * Dk + c] / std::sqrt(n));
    }
  for (auto& x : v) x = r.normal();
  for (auto& x : g) x = float(std::exp(-std::fmin(8.0, std::log1p(std::exp(double(r.normal()))))));
  for (auto& x : beta) x = float(1.0 / (1.0 + std::exp(-double(r.normal()))));
  for (auto& x : s0) x = 0.1f * r.normal();
  for (auto& x : dy) x = r.normal();
  for (auto& x : ds) x = 0.1f * r.normal();

  const Tensor tq = make(q, {B, T, Hk, Dk}, dt), tk = make(k, {B, T, Hk, Dk}, dt), tv = make(v, {B, T, Hv, Dv}, dt);
  const Tensor tg = make(g, {B, T, Hv}, qb::float32), tb = make(beta, {B, T, Hv}, dt);
  const Tensor ts = make(s0, {B, Hv, Dv, Dk}, qb::float32), tdy = make(dy, {B, T, Hv, Dv}, dt);
  const Tensor tds = make(ds, {B, Hv, Dv, Dk}, qb::float32);

  gdn_ref_shape sh{B, T, Hk, Hv, Dk, Dv, 64, 0, nullptr, 0};
  std::vector<float> y(nv), st(ns), ck(size_t(gdn_ref_num_chunks(&sh)) * Hv * Dv * Dk);
  gdn_ref_fwd_f32(&sh, tq.host.data(), tk.host.data(), tv.host.data(), tg.host.data(), tb.host.data(),
                  ts.host.data(), y.data(), st.data(), ck.data());
  std::vector<float> dq(nqk), dk(nqk), dv(nv), dg(ng), db(ng), ds0(ns);
  gdn_ref_bwd_f32(&sh, tq.host.data(), tk.host.data(), tv.host.data(), tg.host.data(), tb.host.data(), ck.data(),
                  tdy.host.data(), tds.host.data(), dq.data(), dk.data(), dv.data(), dg.data(), db.data(),
                  ds0.data());

  for (int train = 0; train < 2; ++train) {
    auto [yo, so] = qb::gated_delta(tq.dev, tk.dev, tv.dev, tg.dev, tb.dev, ts.dev, train != 0);
    std::printf(" gated_delta(train=%d)\n", train);
    if (yo.dtype() != tq.dev.dtype()) std::printf("  y dtype differs from q's  <-- FAIL\n"), ++failures;
    compare("y", yo, y, 2e-3);
    compare("S_T", so, st, 2e-3);
  }
  std::printf(" gated_delta_vjp\n");
  const std::vector<qb::array> gr =
      qb::gated_delta_vjp({tq.dev, tk.dev, tv.dev, tg.dev, tb.dev, ts.dev}, tdy.dev, tds.dev);
  const char* names[6] = {"dq", "dk", "dv", "dg", "dbeta", "dS0"};
  const std::vector<float>* refs[6] = {&dq, &dk, &dv, &dg, &db, &ds0};
  for (int i = 0; i < 6; ++i) compare(names[i], gr[i], *refs[i], 2e-3);

  // The state after every token: the oracle's checkpoints at stride 1 (the state before each token), shifted by one.
  std::printf(" gated_delta_rows\n");
  gdn_ref_shape sh1{B, T, Hk, Hv, Dk, Dv, 1, 0, nullptr, 0};
  std::vector<float> y1(nv), st1(ns), ck1(size_t(gdn_ref_num_chunks(&sh1)) * Hv * Dv * Dk);
  gdn_ref_fwd_f32(&sh1, tq.host.data(), tk.host.data(), tv.host.data(), tg.host.data(), tb.host.data(),
                  ts.host.data(), y1.data(), st1.data(), ck1.data());
  const size_t S = size_t(Hv) * Dv * Dk;
  std::vector<float> rows_ref(size_t(B) * T * S);
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      const float* src = t + 1 < T ? &ck1[(size_t(b) * T + t + 1) * S] : &st1[size_t(b) * S];
      std::memcpy(&rows_ref[(size_t(b) * T + t) * S], src, S * sizeof(float));
    }
  auto [yr, rows] = qb::gated_delta_rows(tq.dev, tk.dev, tv.dev, tg.dev, tb.dev, ts.dev);
  compare("y", yr, y1, 2e-3);
  compare("rows", rows, rows_ref, 2e-3);
}

double sig(double x) { return 1.0 / (1.0 + std::exp(-x)); }

// The neighbours in float32 against their formulas in float64 (src/deltanet.cpp:22-45, 94-100, 122).
void neighbours_case() {
  const int B = 2, T = 37, Hk = 2, Hv = 4, D = 64;
  std::printf("case neighbours: B=%d T=%d Hk=%d Hv=%d D=%d f32\n", B, T, Hk, Hv, D);
  Rng r{21};
  const size_t nqk = size_t(B) * T * Hk * D, ng = size_t(B) * T * Hv, ny = size_t(B) * T * Hv * D;
  auto fill = [&](size_t n, double sc, double mean = 0.0) {
    std::vector<float> x(n);
    for (auto& e : x) e = float(mean + sc * r.normal());
    return x;
  };
  const std::vector<float> qr = fill(nqk, 1), kr = fill(nqk, 1), a = fill(ng, 1), b = fill(ng, 1);
  std::vector<float> alog(Hv), dt = fill(Hv, 0.5);
  for (auto& e : alog) e = float(std::log(1.0 + 15.0 * r.uniform()));
  const std::vector<float> gq = fill(nqk, 1), gk = fill(nqk, 1), gb = fill(ng, 1), gl = fill(ng, 1);
  const std::vector<float> y = fill(ny, 0.05), z = fill(ny, 2), w = fill(D, 0.2, 1.0), go = fill(ny, 1);
  const qb::Dtype f = qb::float32;
  auto dev = [&](const std::vector<float>& x, qb::Shape s) { return qb::array::from_host(x.data(), s, f); };
  const qb::Shape sqk{B, T, Hk, D}, sg{B, T, Hv}, sy{B, T, Hv, D};
  // Row statistics: rho = (mean x^2 + eps)^-1/2 per row of D.
  auto rho = [&](const std::vector<float>& x, size_t row, double eps) {
    double ss = 0;
    for (int c = 0; c < D; ++c) ss += double(x[row * D + c]) * x[row * D + c];
    return 1.0 / std::sqrt(ss / D + eps);
  };
  const double s_q = float(1.0 / D), s_k = float(1.0 / std::sqrt(double(D)));
  std::vector<float> q(nqk), k(nqk), dqr(nqk), dkr(nqk), beta(ng), ld(ng), da(ng), db(ng), dal(Hv, 0.f), ddt(Hv, 0.f);
  for (size_t row = 0; row < nqk / D; ++row)
    for (int which = 0; which < 2; ++which) {
      const std::vector<float>& x = which ? kr : qr;
      const std::vector<float>& gx = which ? gk : gq;
      const double s = which ? s_k : s_q, rh = rho(x, row, 1e-6);
      double sgx = 0;
      for (int c = 0; c < D; ++c) sgx += s * gx[row * D + c] * x[row * D + c];
      for (int c = 0; c < D; ++c) {
        const size_t i = row * D + c;
        (which ? k : q)[i] = float(s * x[i] * rh);
        (which ? dkr : dqr)[i] = float(rh * s * gx[i] - rh * rh * rh * x[i] * sgx / D);
      }
    }
  std::vector<double> dal64(Hv, 0.0), ddt64(Hv, 0.0);
  for (size_t i = 0; i < ng; ++i) {
    const int h = int(i % Hv);
    const double x = double(a[i]) + dt[h], sp = std::log1p(std::exp(-std::fabs(x))) + std::fmax(x, 0.0);
    const double ea = std::exp(double(alog[h])), sb = sig(b[i]);
    beta[i] = float(sb), ld[i] = float(-ea * sp);
    db[i] = float(gb[i] * sb * (1 - sb));
    const double dx = -double(gl[i]) * ea * sig(x);
    da[i] = float(dx);
    dal64[h] += double(gl[i]) * (-ea * sp), ddt64[h] += dx;
  }
  for (int h = 0; h < Hv; ++h) dal[h] = float(dal64[h]), ddt[h] = float(ddt64[h]);
  std::vector<float> o(ny), dy(ny), dz(ny), dw(D, 0.f);
  std::vector<double> dw64(D, 0.0);
  for (size_t row = 0; row < ny / D; ++row) {
    const double rh = rho(y, row, 1e-6);
    double sgy = 0;
    for (int c = 0; c < D; ++c) {
      const size_t i = row * D + c;
      const double zz = z[i], sz = sig(zz), nh = y[i] * rh, dn = go[i] * zz * sz;
      o[i] = float(zz * sz * w[c] * nh);
      dz[i] = float(go[i] * nh * w[c] * sz * (1 + zz * (1 - sz)));
      dw64[c] += dn * nh;
      sgy += dn * w[c] * y[i];
    }
    for (int c = 0; c < D; ++c) {
      const size_t i = row * D + c;
      const double dn = go[i] * double(z[i]) * sig(z[i]);
      dy[i] = float(rh * dn * w[c] - rh * rh * rh * y[i] * sgy / D);
    }
  }
  for (int c = 0; c < D; ++c) dw[c] = float(dw64[c]);

  const qb::array Aqr = dev(qr, sqk), Akr = dev(kr, sqk), Aa = dev(a, sg), Ab = dev(b, sg);
  const qb::array Aal = dev(alog, {Hv}), Adt = dev(dt, {Hv});
  std::printf(" deltanet_prologue\n");
  const qb::Prologue P = qb::deltanet_prologue(Aqr, Akr, Aa, Ab, Aal, Adt);
  compare("q", P.q, q, 1e-5), compare("k", P.k, k, 1e-5), compare("beta", P.beta, beta, 1e-5);
  compare("logdec", P.log_decay, ld, 1e-5);
  std::printf(" deltanet_prologue_vjp\n");
  const qb::PrologueGrads G =
      qb::deltanet_prologue_vjp(Aqr, Akr, Aa, Ab, Aal, Adt, dev(gq, sqk), dev(gk, sqk), dev(gb, sg), dev(gl, sg));
  compare("dq_raw", G.dq_raw, dqr, 1e-5), compare("dk_raw", G.dk_raw, dkr, 1e-5);
  compare("da", G.da, da, 1e-5), compare("db", G.db, db, 1e-5);
  compare("dA_log", G.da_log, dal, 1e-4), compare("ddt", G.ddt_bias, ddt, 1e-4);
  const qb::array Ay = dev(y, sy), Az = dev(z, sy), Aw = dev(w, {D});
  std::printf(" deltanet_epilogue\n");
  compare("o", qb::deltanet_epilogue(Ay, Az, Aw, 1e-6f), o, 1e-5);
  std::printf(" deltanet_epilogue_vjp\n");
  const qb::EpilogueGrads E = qb::deltanet_epilogue_vjp(Ay, Az, Aw, 1e-6f, dev(go, sy));
  compare("dy", E.dy, dy, 1e-5), compare("dz", E.dz, dz, 1e-5), compare("dw", E.dnorm_w, dw, 1e-4);
}

void same(const char* what, const qb::array& a, const qb::array& b) {
  const std::vector<float> x = fetch(a), y = fetch(b);
  const bool ok = x.size() == y.size() && std::memcmp(x.data(), y.data(), x.size() * sizeof(float)) == 0;
  std::printf("  %-8s bit-equal%s\n", what, ok ? "" : "  <-- FAIL");
  failures += !ok;
}

// The prologue fused into the recurrence against the separate steps: deltanet_prologue, then the chunked forward
// and backward through the C ABI with the log-decay (g_is_log = 1), then deltanet_prologue_vjp. Every output but
// the summed gate-parameter cotangents must be the same bits; those two differ by float32 reassociation only.
void fused_case() {
  const int B = 2, T = 150, Hk = 2, Hv = 4, Dk = 128, Dv = 64;
  std::printf("case prologue + recurrence: B=%d T=%d Hk=%d Hv=%d Dk=%d Dv=%d bf16, nonzero state\n", B, T, Hk, Hv, Dk,
              Dv);
  Rng r{31};
  auto fill = [&](size_t n, double sc, double mean = 0.0) {
    std::vector<float> x(n);
    for (auto& e : x) e = float(mean + sc * r.normal());
    return x;
  };
  const qb::Shape sqk{B, T, Hk, Dk}, sv{B, T, Hv, Dv}, sg{B, T, Hv}, ss{B, Hv, Dv, Dk};
  const size_t nqk = size_t(B) * T * Hk * Dk, nv = size_t(B) * T * Hv * Dv, ng = size_t(B) * T * Hv,
               ns = size_t(B) * Hv * Dv * Dk;
  const qb::Dtype bf = qb::bfloat16, f = qb::float32;
  const Tensor qr = make(fill(nqk, 1), sqk, bf), kr = make(fill(nqk, 1), sqk, bf), v = make(fill(nv, 1), sv, bf);
  const Tensor a = make(fill(ng, 1), sg, bf), b = make(fill(ng, 1), sg, bf), dy = make(fill(nv, 1), sv, bf);
  std::vector<float> alog(Hv);
  for (auto& e : alog) e = float(std::log(1.0 + 15.0 * r.uniform()));
  const Tensor al = make(alog, {Hv}, f), dt = make(fill(Hv, 0.5), {Hv}, f);
  const Tensor s0 = make(fill(ns, 0.02), ss, f), dso = make(fill(ns, 1), ss, f);

  std::printf(" deltanet_prologue_recurrence\n");
  const qb::PrologueRecurrence F = qb::deltanet_prologue_recurrence(qr.dev, kr.dev, v.dev, a.dev, b.dev, al.dev,
                                                                    dt.dev, s0.dev);
  const qb::Prologue P = qb::deltanet_prologue(qr.dev, kr.dev, a.dev, b.dev, al.dev, dt.dev);
  qb_gdn_desc d{};
  d.B = B, d.T = T, d.Hk = Hk, d.Hv = Hv, d.Dk = Dk, d.Dv = Dv, d.chunk = 64, d.dtype = QB_DTYPE_BF16, d.g_is_log = 1;
  d.design = QB_GDN_CHUNKED;
  char err[512];
  auto buf = [](size_t bytes) { return qb::array({int((bytes + 3) / 4) + 1}, qb::float32); };
  qb::array ckpt = buf(qb_gdn_ckpt_bytes(&d)), ws = buf(qb_gdn_workspace_bytes(&d));
  qb::array y(sv, bf), s_out(ss, f);
  auto abi = [&](int rc) {
    if (rc != 0) {
      std::printf("  C ABI call failed: %s  <-- FAIL\n", err);
      ++failures;
    }
  };
  abi(qb_gdn_fwd(&d, P.q.data(), P.k.data(), v.dev.data(), static_cast<const float*>(P.log_decay.data()),
                 P.beta.data(), static_cast<const float*>(s0.dev.data()), y.data(), static_cast<float*>(s_out.data()),
                 static_cast<float*>(ckpt.data()), ws.data(), qb::stream(), err, sizeof err));
  same("y", F.y, y), same("state", F.state, s_out), same("q", F.q, P.q), same("k", F.k, P.k);
  same("beta", F.beta, P.beta), same("logdec", F.log_decay, P.log_decay);

  std::printf(" deltanet_prologue_recurrence_vjp\n");
  const qb::PrologueRecurrenceGrads G = qb::deltanet_prologue_recurrence_vjp(
      qr.dev, kr.dev, v.dev, a.dev, b.dev, al.dev, dt.dev, s0.dev, dy.dev, dso.dev);
  qb::array dq(sqk, bf), dk(sqk, bf), dv(sv, bf), dl(sg, f), dbeta(sg, bf), ds0(ss, f);
  abi(qb_gdn_bwd(&d, P.q.data(), P.k.data(), v.dev.data(), static_cast<const float*>(P.log_decay.data()),
                 P.beta.data(), static_cast<const float*>(ckpt.data()), dy.dev.data(),
                 static_cast<const float*>(dso.dev.data()), dq.data(), dk.data(), dv.data(),
                 static_cast<float*>(dl.data()), dbeta.data(), static_cast<float*>(ds0.data()), ws.data(), qb::stream(),
                 err, sizeof err));
  const qb::PrologueGrads S = qb::deltanet_prologue_vjp(qr.dev, kr.dev, a.dev, b.dev, al.dev, dt.dev, dq, dk, dbeta, dl);
  same("dq_raw", G.dq_raw, S.dq_raw), same("dk_raw", G.dk_raw, S.dk_raw), same("dv", G.dv, dv);
  same("da", G.da, S.da), same("db", G.db, S.db), same("dstate", G.dstate, ds0);
  compare("dA_log", G.da_log, fetch(S.da_log), 1e-5), compare("ddt", G.ddt_bias, fetch(S.ddt_bias), 1e-5);
}

void expect_throw(const char* what, void (*fn)()) {
  try {
    fn();
    std::printf("  %s: no exception  <-- FAIL\n", what);
    ++failures;
  } catch (const std::runtime_error& e) {
    std::printf("  %s: runtime_error \"%s\"\n", what, e.what());
  }
}

}  // namespace

int main() {
  run_case("chunked", 2, 150, 2, 4, 128, 64, qb::bfloat16, 11);
  run_case("recurrent", 1, 100, 2, 4, 64, 32, qb::float32, 12);
  neighbours_case();
  fused_case();
  std::printf("errors\n");
  expect_throw("k shape", [] {
    const qb::array q = qb::array::zeros({1, 8, 2, 64}, qb::float32), k = qb::array::zeros({1, 8, 2, 32}, qb::float32);
    const qb::array v = qb::array::zeros({1, 8, 2, 64}, qb::float32), g = qb::array::zeros({1, 8, 2}, qb::float32);
    const qb::array s = qb::array::zeros({1, 2, 64, 64}, qb::float32);
    qb::gated_delta(q, k, v, g, g, s);
  });
  expect_throw("Hv % Hk", [] {
    const qb::array q = qb::array::zeros({1, 8, 2, 64}, qb::float32), v = qb::array::zeros({1, 8, 3, 64}, qb::float32);
    const qb::array g = qb::array::zeros({1, 8, 3}, qb::float32), s = qb::array::zeros({1, 3, 64, 64}, qb::float32);
    qb::gated_delta(q, q, v, g, g, s);
  });
  expect_throw("vjp primals", [] { qb::gated_delta_vjp({}, qb::array(), qb::array()); });
  expect_throw("prologue Dk", [] {
    const qb::array x = qb::array::zeros({1, 8, 2, 32}, qb::float32), a = qb::array::zeros({1, 8, 4}, qb::float32);
    const qb::array p = qb::array::zeros({4}, qb::float32);
    qb::deltanet_prologue(x, x, a, a, p, p);
  });
  expect_throw("fused prologue dtype", [] {
    const qb::array x = qb::array::zeros({1, 8, 2, 128}, qb::float32), a = qb::array::zeros({1, 8, 4}, qb::float32);
    const qb::array v = qb::array::zeros({1, 8, 4, 64}, qb::float32), p = qb::array::zeros({4}, qb::float32);
    qb::deltanet_prologue_recurrence(x, x, v, a, a, p, p, qb::array());
  });
  expect_throw("epilogue weight", [] {
    const qb::array y = qb::array::zeros({1, 8, 4, 64}, qb::float32), w = qb::array::zeros({32}, qb::float32);
    qb::deltanet_epilogue(y, y, w, 1e-6f);
  });
  std::printf(failures ? "FAIL (%d)\n" : "PASS\n", failures);
  return failures ? 1 : 0;
}
