// Small-vector, quaternion and SO(3) math for the AVBD step, usable on the
// host and on gfx950.  The arithmetic order of every expression follows the
// reference core (src/cuda/kernel.cuh:86-228) so that float32 and float64
// results track the reference's CPU build to rounding; in the float build the
// reference evaluates a few expressions in double (its literals are double),
// and the same expressions are evaluated in double here (marked [double]).
// Vector division multiplies by the reciprocal, as kernel.cuh:100 does.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>

#define DUCK_HD __host__ __device__ __forceinline__

namespace duckhip {

// Precision-explicit libm / OCML entry points.
DUCK_HD float msqrt(float x) { return sqrtf(x); }
DUCK_HD double msqrt(double x) { return sqrt(x); }
DUCK_HD float msin(float x) { return sinf(x); }
DUCK_HD double msin(double x) { return sin(x); }
DUCK_HD float mcos(float x) { return cosf(x); }
DUCK_HD double mcos(double x) { return cos(x); }
DUCK_HD float matan2(float y, float x) { return atan2f(y, x); }
DUCK_HD double matan2(double y, double x) { return atan2(y, x); }
DUCK_HD float mhypot(float x, float y) { return hypotf(x, y); }
DUCK_HD double mhypot(double x, double y) { return hypot(x, y); }
// double(hypot(dx, dy)) < .005 as the host's float hypot decides it: that
// hypot rounds the double square root of the double sum of squares to
// float, and the float squares are exact in double, so the test is one
// threshold on that sum -- the smallest sum whose rounded root is not below
// .005, found by bisection over the doubles.
DUCK_HD bool withinFiveMm(float dx, float dy) {
  return double(dx) * double(dx) + double(dy) * double(dy) < 0x1.a36e30068db92p-16;
}
DUCK_HD bool withinFiveMm(double dx, double dy) { return hypot(dx, dy) < .005; }
DUCK_HD float mabs(float x) { return fabsf(x); }
DUCK_HD double mabs(double x) { return fabs(x); }
DUCK_HD bool mfinite(float x) { return __builtin_isfinite(x); }
DUCK_HD bool mfinite(double x) { return __builtin_isfinite(x); }
// Bitwise equality (distinguishes -0 from +0; a NaN equals its own bits).
DUCK_HD bool sameBits(float a, float b) {
  return __builtin_bit_cast(unsigned, a) == __builtin_bit_cast(unsigned, b);
}
DUCK_HD bool sameBits(double a, double b) {
  return __builtin_bit_cast(unsigned long long, a) == __builtin_bit_cast(unsigned long long, b);
}

// Solver arithmetic.  The float solver uses the gfx950 reciprocal, square
// root and reciprocal square root instructions (about 1 ulp) instead of the
// correctly rounded multi-instruction sequences; the double solver keeps the
// correctly rounded operations and so tracks the float64 oracle to rounding.
// Only the block solve, predictor and velocity recovery use these; contact
// detection and colouring keep the exact operations (their outputs are
// discrete and must not move).
DUCK_HD float frcp(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_rcpf(x);
#else
  return 1.0f / x;
#endif
}
DUCK_HD double frcp(double x) { return 1.0 / x; }
DUCK_HD float fsqrt(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_sqrtf(x);
#else
  return sqrtf(x);
#endif
}
DUCK_HD double fsqrt(double x) { return sqrt(x); }
DUCK_HD float frsqrt(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_rsqf(x);
#else
  return 1.0f / sqrtf(x);
#endif
}
DUCK_HD double frsqrt(double x) { return 1.0 / sqrt(x); }
// a * b + c.  The float solver fuses it (one rounding, v_fma_f32; the
// reference's own CUDA build keeps the two roundings, --fmad=false in
// scripts/build_cuda.py:37, so the float results differ from it by rounding);
// in double it is the separately rounded a * b + c, so every solver expression
// written with fmad keeps the float64 oracle's operation order and rounding
// exactly.
DUCK_HD float fmad(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
DUCK_HD double fmad(double a, double b, double c) { return a * b + c; }
// |(x, y)|: the hardware square root of x^2 + y^2 in float (solver
// magnitudes are far from overflow), hypot in double.
DUCK_HD float fhypot(float x, float y) { return fsqrt(fmad(x, x, y * y)); }
DUCK_HD double fhypot(double x, double y) { return hypot(x, y); }
// a / b: a * rcp(b) in float, a true division in double.
DUCK_HD float fdiv(float a, float b) { return a * frcp(b); }
DUCK_HD double fdiv(double a, double b) { return a / b; }
// a / b given inv = frcp(b): the float path multiplies, the double path divides.
DUCK_HD float fdivInv(float a, float, float inv) { return a * inv; }
DUCK_HD double fdivInv(double a, double b, double) { return a / b; }

template <class R> struct V3 {
  R x, y, z;
};
template <class R> struct Q4 {
  R w, x, y, z;
};

template <class R> DUCK_HD V3<R> v3(R x, R y, R z) { return V3<R>{x, y, z}; }
template <class R> DUCK_HD V3<R> operator+(V3<R> a, V3<R> b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
template <class R> DUCK_HD V3<R> operator-(V3<R> a, V3<R> b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
template <class R> DUCK_HD V3<R> operator-(V3<R> a) { return {-a.x, -a.y, -a.z}; }
template <class R> DUCK_HD V3<R> operator*(V3<R> a, R s) { return {a.x * s, a.y * s, a.z * s}; }
template <class R> DUCK_HD V3<R> operator*(R s, V3<R> a) { return {a.x * s, a.y * s, a.z * s}; }
template <class R> DUCK_HD V3<R> divide(V3<R> a, R s) { return a * (R(1) / s); }
template <class R> DUCK_HD R dot(V3<R> a, V3<R> b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
template <class R> DUCK_HD V3<R> cross(V3<R> a, V3<R> b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
template <class R> DUCK_HD R norm(V3<R> a) { return msqrt(dot(a, a)); }
template <class R> DUCK_HD R comp(V3<R> a, int k) { return k == 0 ? a.x : (k == 1 ? a.y : a.z); }
template <class R> DUCK_HD V3<R> unitOrNan(V3<R> a) {
  R n = norm(a);
  if (double(n) < 1e-15)
    return {R(NAN), R(NAN), R(NAN)};
  return divide(a, n);
}

template <class R> DUCK_HD Q4<R> conj(Q4<R> q) { return {q.w, -q.x, -q.y, -q.z}; }
template <class R> DUCK_HD Q4<R> operator*(Q4<R> a, Q4<R> b) {
  return {a.w * b.w - a.x * b.x - a.y * b.y - a.z * b.z,
          a.w * b.x + a.x * b.w + a.y * b.z - a.z * b.y,
          a.w * b.y - a.x * b.z + a.y * b.w + a.z * b.x,
          a.w * b.z + a.x * b.y - a.y * b.x + a.z * b.w};
}
template <class R> DUCK_HD Q4<R> normalized(Q4<R> q) {
  R n = msqrt(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  if (double(n) < 1e-15)
    return {R(NAN), R(NAN), R(NAN), R(NAN)};
  return {q.w / n, q.x / n, q.y / n, q.z / n};
}
// v + 2 u x (u x v + w v)
template <class R> DUCK_HD V3<R> rotate(Q4<R> q, V3<R> v) {
  V3<R> u{q.x, q.y, q.z};
  return v + R(2) * cross(u, cross(u, v) + q.w * v);
}
// Rotation by the conjugate, without forming it (bitwise equal to
// rotate(conj(q), v): negating u flips both cross products).
template <class R> DUCK_HD V3<R> rotateInv(Q4<R> q, V3<R> v) { return rotate(conj(q), v); }

template <class R> DUCK_HD Q4<R> expmap(V3<R> v) {
  R a = norm(v), s;
  if (double(a) < 1e-8)
    s = R(0.5 - double(a * a / R(48))); // [double]
  else
    s = msin(a / R(2)) / a;
  return normalized(Q4<R>{mcos(a / R(2)), s * v.x, s * v.y, s * v.z});
}
template <class R> DUCK_HD V3<R> logmap(Q4<R> q) {
  q = normalized(q);
  if (q.w < 0)
    q = {-q.w, -q.x, -q.y, -q.z};
  V3<R> v{q.x, q.y, q.z};
  R s = norm(v);
  R k = double(s) < 1e-10 ? R(2) : R(2) * matan2(s, q.w) / s;
  return v * k;
}

// Solver forms of dot, cross, x + s v, rotation and the quaternion product,
// written with fmad: fused in float; in double the same operations in the
// same order as dot / cross / operator* / rotate above, so bitwise equal.
template <class R> DUCK_HD R fdot(V3<R> a, V3<R> b) { return fmad(a.z, b.z, fmad(a.y, b.y, a.x * b.x)); }
template <class R> DUCK_HD V3<R> fcross(V3<R> a, V3<R> b) {
  return {fmad(a.y, b.z, -(a.z * b.y)), fmad(a.z, b.x, -(a.x * b.z)), fmad(a.x, b.y, -(a.y * b.x))};
}
template <class R> DUCK_HD V3<R> faxpy(R s, V3<R> v, V3<R> x) {
  return {fmad(s, v.x, x.x), fmad(s, v.y, x.y), fmad(s, v.z, x.z)};
}
template <class R> DUCK_HD V3<R> frotate(Q4<R> q, V3<R> v) {
  V3<R> u{q.x, q.y, q.z};
  return faxpy(R(2), fcross(u, faxpy(q.w, v, fcross(u, v))), v);
}
template <class R> DUCK_HD Q4<R> fqmul(Q4<R> a, Q4<R> b) {
  return {fmad(-a.z, b.z, fmad(-a.y, b.y, fmad(-a.x, b.x, a.w * b.w))),
          fmad(-a.z, b.y, fmad(a.y, b.z, fmad(a.x, b.w, a.w * b.x))),
          fmad(a.z, b.x, fmad(a.y, b.w, fmad(-a.x, b.z, a.w * b.y))),
          fmad(a.z, b.w, fmad(-a.y, b.x, fmad(a.x, b.y, a.w * b.z)))};
}

// atan2 for the float solver (exact atan2 for double): reduction to
// t = min(|x|, |y|) / max(|x|, |y|) in [0, 1], atan(t) = t P(t^2) with P of
// degree 8 fitted to minimise the maximum error on [0, 1] (5.8e-9 rad before
// float rounding), then the octant and sign.  atan2(0, 0) gives 0.
DUCK_HD float fatan2(float y, float x) {
  const float ax = fabsf(x), ay = fabsf(y);
  const float hi = ax > ay ? ax : ay, lo = ax > ay ? ay : ax;
  const float t = hi > 0 ? lo * frcp(hi) : 0.0f, t2 = t * t;
  float p = fmad(t2, 0.002456715321358685f, -0.014401324459861229f);
  p = fmad(t2, p, 0.03978117660090867f);
  p = fmad(t2, p, -0.07234854241710113f);
  p = fmad(t2, p, 0.10498945199758145f);
  p = fmad(t2, p, -0.14161229220755356f);
  p = fmad(t2, p, 0.19985906832392586f);
  p = fmad(t2, p, -0.3333259703951586f);
  p = fmad(t2, p, 0.9999998863880095f);
  float r = t * p;
  r = ay > ax ? 1.5707963267948966f - r : r;
  r = x < 0 ? 3.14159265358979323846f - r : r;
  return copysignf(r, y);
}
DUCK_HD double fatan2(double y, double x) { return matan2(y, x); }

// Fast forms of norm / normalized / expmap / logmap for the float solver
// (exact forms for double).  Small rotations, the common case inside the
// block solve, use truncated Taylor series whose first omitted term is below
// 1e-11 relative on the stated ranges.
template <class R> DUCK_HD R fnorm(V3<R> a) { return fsqrt(fdot(a, a)); }
template <class R> DUCK_HD Q4<R> fnormalized(Q4<R> q) {
  if constexpr (sizeof(R) == sizeof(float)) {
    R n2 = fmad(q.z, q.z, fmad(q.y, q.y, fmad(q.x, q.x, q.w * q.w)));
    if (double(n2) < 1e-30)
      return {R(NAN), R(NAN), R(NAN), R(NAN)};
    R inv = frsqrt(n2);
    return {q.w * inv, q.x * inv, q.y * inv, q.z * inv};
  } else {
    return normalized(q);
  }
}
template <class R> DUCK_HD Q4<R> fexpmap(V3<R> v) {
  if constexpr (sizeof(R) == sizeof(float)) {
    R a = fnorm(v), s, c;
    if (a < R(0.25)) {
      R a2 = a * a;
      // sin(a/2)/a and cos(a/2)
      s = fmad(a2, fmad(a2, fmad(a2, R(-1.0 / 645120), R(1.0 / 3840)), R(-1.0 / 48)), R(0.5));
      c = fmad(a2, fmad(a2, fmad(a2, fmad(a2, R(1.0 / 10321920), R(-1.0 / 46080)), R(1.0 / 384)),
                        R(-0.125)),
               R(1));
    } else {
      s = msin(a / R(2)) / a;
      c = mcos(a / R(2));
    }
    return fnormalized(Q4<R>{c, s * v.x, s * v.y, s * v.z});
  } else {
    return expmap(v);
  }
}
template <class R> DUCK_HD V3<R> flogmap(Q4<R> q) {
  if constexpr (sizeof(R) == sizeof(float)) {
    q = fnormalized(q);
    if (q.w < 0)
      q = {-q.w, -q.x, -q.y, -q.z};
    V3<R> v{q.x, q.y, q.z};
    R s = fnorm(v), k;
    if (double(s) < 1e-10) {
      k = R(2);
    } else if (q.w > R(0.99)) {
      // 2 atan(s/w)/s = (2/w) atan(t)/t with t = s/w < 0.143
      R iw = frcp(q.w), t = s * iw, t2 = t * t;
      R p = fmad(t2, fmad(t2, fmad(t2, fmad(t2, fmad(t2, R(-1.0 / 11), R(1.0 / 9)), R(-1.0 / 7)), R(0.2)),
                          R(-1.0 / 3)),
                 R(1));
      k = (R(2) * iw) * p;
    } else {
      k = R(2) * matan2(s, q.w) / s;
    }
    return v * k;
  } else {
    return logmap(q);
  }
}

// Rotation matrix (row-major) of a unit quaternion, and its product with v
// (float solver only, fused).
template <class R> DUCK_HD void quatMatrix(Q4<R> q, R m[9]) {
  const R xx = q.x * q.x, yy = q.y * q.y, zz = q.z * q.z;
  const R xy = q.x * q.y, xz = q.x * q.z, yz = q.y * q.z;
  m[0] = fmad(R(-2), yy + zz, R(1));
  m[1] = R(2) * fmad(-q.w, q.z, xy);
  m[2] = R(2) * fmad(q.w, q.y, xz);
  m[3] = R(2) * fmad(q.w, q.z, xy);
  m[4] = fmad(R(-2), xx + zz, R(1));
  m[5] = R(2) * fmad(-q.w, q.x, yz);
  m[6] = R(2) * fmad(-q.w, q.y, xz);
  m[7] = R(2) * fmad(q.w, q.x, yz);
  m[8] = fmad(R(-2), xx + yy, R(1));
}
template <class R> DUCK_HD V3<R> matApply(const R m[9], V3<R> v) {
  return {fmad(m[2], v.z, fmad(m[1], v.y, m[0] * v.x)), fmad(m[5], v.z, fmad(m[4], v.y, m[3] * v.x)),
          fmad(m[8], v.z, fmad(m[7], v.y, m[6] * v.x))};
}

// IEEE remainder(a, 2*pi) in double: n = nearest integer of a/(2 pi), then the
// exactly representable a - n 2pi by one fused operation.  [double]
template <class R> DUCK_HD R wrapAngle(R a) {
  // |a| < 3.14159 < pi: the nearest multiple is 0 and fma(-(+-0), 2 pi, d)
  // is d, except that d = -0 yields +0 -- which a + 0 reproduces exactly.
  if (mabs(a) < R(3.14159))
    return a + R(0);
  const double twoPi = 6.283185307179586476925286766559; // 2*acos(-1.0)
  double d = double(a);
  double n = rint(d / twoPi);
  return R(fma(-n, twoPi, d));
}

// Both angles wrapped, with one test for the common case of both already
// inside (-pi, pi).
template <class R> DUCK_HD void wrapAngle2(R a, R b, R &wa, R &wb) {
  if (mabs(a) < R(3.14159) && mabs(b) < R(3.14159)) {
    wa = a + R(0);
    wb = b + R(0);
  } else {
    wa = wrapAngle(a);
    wb = wrapAngle(b);
  }
}

template <class R> DUCK_HD R mn(R a, R b) { return a < b ? a : b; }
template <class R> DUCK_HD R mx(R a, R b) { return a > b ? a : b; }
template <class R> DUCK_HD R clampv(R v, R a, R b) { return mn(mx(v, a), b); }

template <class R> DUCK_HD R hingeAngle(Q4<R> qa, Q4<R> qb, V3<R> axisA, V3<R> tangentA,
                                        V3<R> tangentB) {
  V3<R> axis = rotate(qa, axisA), t = rotate(qa, tangentA), u = rotate(qb, tangentB);
  return matan2(dot(axis, cross(t, u)), dot(t, u));
}

} // namespace duckhip
