// Host build of the solver's math forms (duck_gym_amd/csrc/avbd_math.hpp, avbd_step.hpp),
// printed as "name value" lines for tests/test_solver_math.py.  On the host
// frcp / fsqrt / frsqrt are the correctly rounded operations; the device
// instructions they map to are covered by the GPU parity tests.
#include "avbd_step.hpp"

#include <cstdio>
#include <cstring>
#include <random>

using namespace duckhip;

static bool same(double a, double b) { return std::memcmp(&a, &b, sizeof a) == 0; }

int main() {
  std::mt19937_64 rng(20260927);
  std::uniform_real_distribution<double> u(-1.0, 1.0);

  // fatan2 against atan2 in double over a grid of both signs, and the
  // signed zeros and axes.
  double worst = 0;
  for (int i = 0; i <= 4000; ++i)
    for (int j = 0; j <= 400; ++j) {
      const float y = -1.0f + 2.0f * float(i) / 4000, x = -1.0f + 2.0f * float(j) / 400;
      const double e = std::fabs(double(fatan2(y, x)) - std::atan2(double(y), double(x)));
      worst = e > worst ? e : worst;
    }
  std::printf("atan2_max_error %.9e\n", worst);
  const float cases[][2] = {{0.0f, 1.0f}, {-0.0f, 1.0f}, {0.0f, -1.0f}, {-0.0f, -1.0f}, {1.0f, 0.0f}, {-1.0f, 0.0f}};
  double special = 0;
  for (auto &c : cases) {
    const double e = std::fabs(double(fatan2(c[0], c[1])) - std::atan2(double(c[0]), double(c[1])));
    special = e > special ? e : special;
  }
  std::printf("atan2_special_error %.9e\n", special);

  // Small-rotation series of the float solver against the exact double forms.
  double expErr = 0, logErr = 0, coefErr = 0;
  for (int n = 0; n < 20000; ++n) {
    const double s = 0.24 * double(n % 1000) / 1000;
    V3<double> vd{u(rng), u(rng), u(rng)};
    const double len = std::sqrt(dot(vd, vd));
    vd = vd * (s / (len > 0 ? len : 1));
    const V3<float> vf{float(vd.x), float(vd.y), float(vd.z)};
    const Q4<float> qf = fexpmap(vf);
    const Q4<double> qd = expmap(V3<double>{double(vf.x), double(vf.y), double(vf.z)});
    const double e = std::fmax(std::fmax(std::fabs(qf.w - qd.w), std::fabs(qf.x - qd.x)),
                               std::fmax(std::fabs(qf.y - qd.y), std::fabs(qf.z - qd.z)));
    expErr = e > expErr ? e : expErr;
    const V3<float> lf = flogmap(qf);
    const V3<double> ld = logmap(Q4<double>{double(qf.w), double(qf.x), double(qf.y), double(qf.z)});
    const double le = std::fmax(std::fabs(lf.x - ld.x), std::fmax(std::fabs(lf.y - ld.y), std::fabs(lf.z - ld.z)));
    logErr = le > logErr ? le : logErr;
    const float a = float(2 * s);
    const double ad = double(a);
    const double exact = ad < 1e-5 ? 1.0 / 12 : (1 - 0.5 * ad / std::tan(0.5 * ad)) / (ad * ad);
    const double ce = std::fabs(double(logJacobianCoef(a)) - exact) / exact;
    coefErr = ce > coefErr ? ce : coefErr;
  }
  std::printf("expmap_max_error %.9e\n", expErr);
  std::printf("logmap_max_error %.9e\n", logErr);
  std::printf("logjac_max_rel_error %.9e\n", coefErr);

  // The fused forms are, in double, the reference's operations in the same
  // order: bitwise equal.
  int mismatches = 0;
  for (int n = 0; n < 100000; ++n) {
    const V3<double> a{u(rng), u(rng), u(rng)}, b{u(rng), u(rng), u(rng)};
    const Q4<double> q{u(rng), u(rng), u(rng), u(rng)}, r{u(rng), u(rng), u(rng), u(rng)};
    const double s = u(rng);
    const V3<double> c1 = cross(a, b), c2 = fcross(a, b), r1 = rotate(q, a), r2 = frotate(q, a);
    const V3<double> x1 = a + s * b, x2 = faxpy(s, b, a);
    const Q4<double> m1 = q * r, m2 = fqmul(q, r);
    mismatches += !same(dot(a, b), fdot(a, b));
    mismatches += !same(c1.x, c2.x) + !same(c1.y, c2.y) + !same(c1.z, c2.z);
    mismatches += !same(r1.x, r2.x) + !same(r1.y, r2.y) + !same(r1.z, r2.z);
    mismatches += !same(x1.x, x2.x) + !same(x1.y, x2.y) + !same(x1.z, x2.z);
    mismatches += !same(m1.w, m2.w) + !same(m1.x, m2.x) + !same(m1.y, m2.y) + !same(m1.z, m2.z);
  }
  std::printf("double_fused_mismatches %d\n", mismatches);

  // The float block solve (L D L^T) against the double Cholesky solve on
  // random SPD systems (condition up to ~1e3), and both return NaN on an
  // indefinite one.
  double solveErr = 0;
  int solveNan = 0;
  for (int n = 0; n < 20000; ++n) {
    double A[6][6];
    for (int i = 0; i < 6; ++i)
      for (int j = 0; j < 6; ++j)
        A[i][j] = u(rng);
    Hess<double> hd;
    Hess<float> hf;
    const double ridge = 0.01 + 2.0 * double(n % 100) / 100;
    for (int i = 0; i < 6; ++i) {
      for (int j = 0; j <= i; ++j) {
        double v = i == j ? ridge : 0.0;
        for (int k = 0; k < 6; ++k)
          v += A[i][k] * A[j][k];
        hf.h[tri(i, j)] = float(v);
        hd.h[tri(i, j)] = double(hf.h[tri(i, j)]);
      }
      hf.g[i] = float(u(rng));
      hd.g[i] = double(hf.g[i]);
    }
    float xf[6];
    double xd[6], scale = 0;
    solve6(hf, xf);
    solve6(hd, xd);
    for (int i = 0; i < 6; ++i)
      scale = std::fmax(scale, std::fabs(xd[i]));
    for (int i = 0; i < 6; ++i)
      solveErr = std::fmax(solveErr, std::fabs(double(xf[i]) - xd[i]) / scale);
  }
  {
    Hess<float> hf{};
    Hess<double> hd{};
    for (int i = 0; i < 6; ++i)
      hf.h[tri(i, i)] = hd.h[tri(i, i)] = i == 3 ? -1.0f : 1.0f;
    float xf[6];
    double xd[6];
    solve6(hf, xf);
    solve6(hd, xd);
    for (int i = 0; i < 6; ++i)
      solveNan += std::isnan(xf[i]) && std::isnan(xd[i]);
  }
  std::printf("solve6_float_rel_error %.9e\n", solveErr);
  std::printf("solve6_indefinite_nan %d\n", solveNan);

  // The sparse rotational Jacobian columns against e - (t x e) / 2 + c t x (t x e).
  double jacErr = 0;
  for (int n = 0; n < 100000; ++n) {
    const V3<double> t{0.5 * u(rng), 0.5 * u(rng), 0.5 * u(rng)};
    const double c = 1.0 / 12 + 0.01 * u(rng);
    V3<double> sparse[3];
    rotationJacobianSparse(t, c, sparse);
    for (int k = 0; k < 3; ++k) {
      const V3<double> e = unitAxis<double>(k);
      const V3<double> full = (e - cross(t, e) * 0.5) + cross(t, cross(t, e)) * c;
      jacErr = std::fmax(jacErr, std::fmax(std::fabs(full.x - sparse[k].x),
                                           std::fmax(std::fabs(full.y - sparse[k].y), std::fabs(full.z - sparse[k].z))));
    }
  }
  std::printf("rotation_jacobian_max_error %.9e\n", jacErr);

  // The 5 mm duplicate test of the ground-point passes against the host's
  // own float hypot (the library the oracle calls), on offsets spread over
  // the square and packed within a few ulps of the 5 mm circle.
  std::uniform_real_distribution<float> side(-0.006f, 0.006f), turn(0.0f, 6.2831853f), jitter(-2e-6f, 2e-6f);
  long fiveMm = 0;
  for (int n = 0; n < 4000000; ++n) {
    float dx, dy;
    if (n & 1) {
      dx = side(rng);
      dy = side(rng);
    } else {
      const float a = turn(rng), rr = 0.005f * (1.0f + jitter(rng));
      dx = rr * std::cos(a);
      dy = rr * std::sin(a);
    }
    fiveMm += withinFiveMm(dx, dy) != (double(std::hypot(dx, dy)) < .005);
  }
  const float axis[] = {0.0f, 0.005f, -0.005f, std::nextafter(0.005f, 0.0f), std::nextafter(0.005f, 1.0f)};
  for (float a : axis)
    for (float b : axis)
      fiveMm += withinFiveMm(a, b) != (double(std::hypot(a, b)) < .005);
  std::printf("five_mm_mismatches %ld\n", fiveMm);
  return 0;
}
