// Checks the C++ adapters of include/qb (gated_delta, gated_delta_trainable, gated_delta_vjp) against the oracle,
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
#include "qb/delta_grad.h"
#include "qb/deltanet.h"

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
  std::printf(failures ? "FAIL (%d)\n" : "PASS\n", failures);
  return failures ? 1 : 0;
}
