// Vector, quaternion and 6x6 block math of the duck C++ interface
// (include/duck/math.hpp of duck_gym: the same names, types and meaning).
// Header-only, double precision, host code.
#pragma once
#include <array>
#include <cmath>
#include <stdexcept>

namespace duck {

struct Vec3 {
  double x = 0, y = 0, z = 0;
  double &operator[](int i) { return i == 0 ? x : (i == 1 ? y : z); }
  double operator[](int i) const { return i == 0 ? x : (i == 1 ? y : z); }
};

inline Vec3 operator+(Vec3 a, Vec3 b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
inline Vec3 operator-(Vec3 a, Vec3 b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
inline Vec3 operator-(Vec3 a) { return {-a.x, -a.y, -a.z}; }
inline Vec3 operator*(Vec3 a, double s) { return {s * a.x, s * a.y, s * a.z}; }
inline Vec3 operator*(double s, Vec3 a) { return a * s; }
inline Vec3 operator/(Vec3 a, double s) { return a * (1 / s); }
inline Vec3 &operator+=(Vec3 &a, Vec3 b) { return a = a + b; }
inline double dot(Vec3 a, Vec3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
inline Vec3 cross(Vec3 a, Vec3 b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
inline double norm(Vec3 a) { return std::sqrt(dot(a, a)); }
// a / |a|; throws std::runtime_error("Zero direction") for |a| < 1e-15.
inline Vec3 unit(Vec3 a) {
  const double n = norm(a);
  if (n < 1e-15)
    throw std::runtime_error("Zero direction");
  return a / n;
}

// Unit quaternion w + (x, y, z); identity by default.
struct Quat {
  double w = 1, x = 0, y = 0, z = 0;
};

inline Quat conjugate(Quat q) { return {q.w, -q.x, -q.y, -q.z}; }
// Hamilton product: rotation b followed by rotation a.
inline Quat operator*(Quat a, Quat b) {
  const Vec3 u{a.x, a.y, a.z}, v{b.x, b.y, b.z};
  const Vec3 c = cross(u, v) + u * b.w + v * a.w;
  return {a.w * b.w - dot(u, v), c.x, c.y, c.z};
}
// q / |q|; throws std::runtime_error("Zero quaternion") for |q| < 1e-15.
inline Quat normalized(Quat q) {
  const double n = std::sqrt(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  if (n < 1e-15)
    throw std::runtime_error("Zero quaternion");
  return {q.w / n, q.x / n, q.y / n, q.z / n};
}
// q v q^-1 for a unit q, as v + 2 u x (u x v + w v).
inline Vec3 rotate(Quat q, Vec3 v) {
  const Vec3 u{q.x, q.y, q.z};
  return v + 2 * cross(u, cross(u, v) + q.w * v);
}
// The rotation by |v| about v / |v| (v a rotation vector).
inline Quat exp(Vec3 v) {
  const double a = norm(v);
  // sin(a/2)/a = 1/2 - a^2/48 + O(a^4)
  const double s = a < 1e-8 ? 0.5 - a * a / 48 : std::sin(0.5 * a) / a;
  return normalized({std::cos(0.5 * a), s * v.x, s * v.y, s * v.z});
}
// The rotation vector of q (angle in [0, pi] after folding to w >= 0).
inline Vec3 log(Quat q) {
  q = normalized(q);
  const double sign = q.w < 0 ? -1 : 1;
  const Vec3 v{sign * q.x, sign * q.y, sign * q.z};
  const double s = norm(v), w = sign * q.w;
  return v * (s < 1e-10 ? 2 : 2 * std::atan2(s, w) / s);
}
// a mod 2 pi into [-pi, pi].
inline double wrap(double a) { return std::remainder(a, 2 * std::acos(-1.0)); }

// Rows of a body's 6-dof system: (translation, rotation).
using V6 = std::array<double, 6>;
using M6 = std::array<V6, 6>;
inline V6 row(Vec3 t, Vec3 r) { return {t.x, t.y, t.z, r.x, r.y, r.z}; }
// g += J force, H += stiffness J J^T.
inline void stamp(M6 &H, V6 &g, const V6 &J, double force, double stiffness) {
  for (int i = 0; i < 6; ++i) {
    g[i] += J[i] * force;
    const double s = stiffness * J[i];
    for (int j = 0; j < 6; ++j)
      H[i][j] += s * J[j];
  }
}
// x with H x = -g for a symmetric positive definite H (its lower triangle is
// read), by Cholesky factorisation; throws std::runtime_error("Non-positive
// local Hessian") on a pivot that is not positive and finite.
inline V6 solve(M6 H, V6 g) {
  M6 L{};
  for (int j = 0; j < 6; ++j) {
    double d = H[j][j];
    for (int k = 0; k < j; ++k)
      d -= L[j][k] * L[j][k];
    if (!(d > 0) || !std::isfinite(d))
      throw std::runtime_error("Non-positive local Hessian");
    L[j][j] = std::sqrt(d);
    for (int i = j + 1; i < 6; ++i) {
      double v = H[i][j];
      for (int k = 0; k < j; ++k)
        v -= L[i][k] * L[j][k];
      L[i][j] = v / L[j][j];
    }
  }
  V6 y{}, x{};
  for (int i = 0; i < 6; ++i) { // L y = -g
    double v = -g[i];
    for (int k = 0; k < i; ++k)
      v -= L[i][k] * y[k];
    y[i] = v / L[i][i];
  }
  for (int i = 5; i >= 0; --i) { // L^T x = y
    double v = y[i];
    for (int k = i + 1; k < 6; ++k)
      v -= L[k][i] * x[k];
    x[i] = v / L[i][i];
  }
  return x;
}

} // namespace duck
