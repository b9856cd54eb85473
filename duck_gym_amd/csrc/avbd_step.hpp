// The AVBD environment step on gfx950: one wave64 workgroup advances
// G = 64 / L environments, L lanes per environment.
//
// Per physics step of one environment (reference: src/cuda/kernel.cuh:937-1095):
//   detection   lanes over shapes (ground manifolds) and pairs (MPR), then a
//               prefix over shapes compacts the contact list in reference order
//   warm start  lanes over joints; predictor lanes over bodies
//   iterations  per colour: lanes over that colour's bodies, each running one
//               6x6 block-descent solve (assembly + LDL^T/Cholesky in registers);
//               then lanes over joints and contacts for the dual/penalty update
//   epilogue    lanes over bodies (velocity recovery), joints and contacts
//               (diagnostics)
// Every __syncthreads() below is reached by all 64 lanes: per-environment
// differences (colour counts, convergence, failure) are masked, never branched
// around a barrier.
#pragma once
#include "avbd_state.hpp"

namespace duckhip {

// StepArgs::motorMode: the controls a launch applies before its steps --
// targets with kp and limit (CudaBatch.step), explicit motor channels
// (step_motor), or none: the state's own (duck_advance).
enum { kTargetControls = 0, kMotorControls = 1, kHeldControls = 2 };

struct StepArgs {
  const void *model;   // DeviceModel<R>
  const void *frames;  // Frames<R, B, J> built from the model (framesKernel)
  const void *points;  // shape points, R[3] each
  unsigned char *states; // EnvState blobs
  long long blobBytes;
  int count;
  const void *targets; // [E,J] or null (step)
  const void *forces;  // [E,3]
  const void *motor;   // [E,J,3] (motor mode)
  int substeps;
  int motorMode; // kTargetControls, kMotorControls or kHeldControls
  double kp, limit;
  int nb, nj, ns, np; // model counts (also in the model), here so that the
                      // first loads need only the kernel arguments
  int bodies;         // read the reset-only block (masses, inertia, friction)
                      // of each state; else they are the model's
};

DUCK_HD constexpr int tri(int i, int j) { return i * (i + 1) / 2 + j; }

template <class R> struct Hess {
  R h[21]; // lower triangle of the 6x6 Hessian
  R g[6];
};

// Row (0, r).
template <class R> DUCK_HD void stampAngular(Hess<R> &H, V3<R> r, R f, R kk) {
  H.g[3] = fmad(r.x, f, H.g[3]);
  H.g[4] = fmad(r.y, f, H.g[4]);
  H.g[5] = fmad(r.z, f, H.g[5]);
  R r0 = kk * r.x, r1 = kk * r.y, r2 = kk * r.z;
  H.h[tri(3, 3)] = fmad(r0, r.x, H.h[tri(3, 3)]);
  H.h[tri(4, 3)] = fmad(r1, r.x, H.h[tri(4, 3)]);
  H.h[tri(4, 4)] = fmad(r1, r.y, H.h[tri(4, 4)]);
  H.h[tri(5, 3)] = fmad(r2, r.x, H.h[tri(5, 3)]);
  H.h[tri(5, 4)] = fmad(r2, r.y, H.h[tri(5, 4)]);
  H.h[tri(5, 5)] = fmad(r2, r.z, H.h[tri(5, 5)]);
}
// General row (t, r).
template <class R> DUCK_HD void stampFull(Hess<R> &H, V3<R> t, V3<R> r, R f, R kk) {
  R J[6] = {t.x, t.y, t.z, r.x, r.y, r.z};
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    H.g[i] = fmad(J[i], f, H.g[i]);
    R ki = kk * J[i];
#pragma unroll
    for (int j = 0; j <= i; ++j)
      H.h[tri(i, j)] = fmad(ki, J[j], H.h[tri(i, j)]);
  }
}
// Row with t = s e_k and r x e_k (a hinge anchor row or a ground-contact
// row): only the entries the unit axis makes non-zero are formed.
template <class R> DUCK_HD void stampAxisRow(Hess<R> &H, int k, R s, V3<R> r, R f, R kk) {
  // r x e_k = (0, z, -y), (-z, 0, x), (y, -x, 0) for k = 0, 1, 2
  R u0 = k == 0 ? R(0) : (k == 1 ? -r.z : r.y);
  R u1 = k == 1 ? R(0) : (k == 0 ? r.z : -r.x);
  R u2 = k == 2 ? R(0) : (k == 0 ? -r.y : r.x);
  H.g[k] = fmad(s, f, H.g[k]);
  H.h[tri(k, k)] += kk;
  R ks = kk * s;
  if (k != 0) {
    H.g[3] = fmad(u0, f, H.g[3]);
    H.h[tri(3, k)] = fmad(ks, u0, H.h[tri(3, k)]);
    H.h[tri(3, 3)] = fmad(kk * u0, u0, H.h[tri(3, 3)]);
  }
  if (k != 1) {
    H.g[4] = fmad(u1, f, H.g[4]);
    H.h[tri(4, k)] = fmad(ks, u1, H.h[tri(4, k)]);
    H.h[tri(4, 4)] = fmad(kk * u1, u1, H.h[tri(4, 4)]);
  }
  if (k != 2) {
    H.g[5] = fmad(u2, f, H.g[5]);
    H.h[tri(5, k)] = fmad(ks, u2, H.h[tri(5, k)]);
    H.h[tri(5, 5)] = fmad(kk * u2, u2, H.h[tri(5, 5)]);
  }
  // the one off-diagonal rotational entry between the two non-zero components
  if (k == 0)
    H.h[tri(5, 4)] = fmad(kk * u2, u1, H.h[tri(5, 4)]);
  else if (k == 1)
    H.h[tri(5, 3)] = fmad(kk * u2, u0, H.h[tri(5, 3)]);
  else
    H.h[tri(4, 3)] = fmad(kk * u1, u0, H.h[tri(4, 3)]);
}

// Column norms, per unit |f|, of 0.5 (r f^T + f r^T) - (r.f) I for f along
// e_k (k = 0, 1, 2): with {i, j} the other two axes, column k is
// 0.5 sqrt(r_i^2 + r_j^2) and column i is sqrt(r_i^2 / 4 + r_k^2).
template <class R> DUCK_HD void axisGeometricNorms(V3<R> r, R g[3][3]) {
  const R q0 = r.x * r.x, q1 = r.y * r.y, q2 = r.z * r.z;
  g[0][0] = R(0.5) * fsqrt(fmad(r.y, r.y, q2));
  g[0][1] = fsqrt(fmad(R(0.25), q1, q0));
  g[0][2] = fsqrt(fmad(R(0.25), q2, q0));
  g[1][0] = fsqrt(fmad(R(0.25), q0, q1));
  g[1][1] = R(0.5) * fsqrt(fmad(r.x, r.x, q2));
  g[1][2] = fsqrt(fmad(R(0.25), q2, q1));
  g[2][0] = fsqrt(fmad(R(0.25), q0, q2));
  g[2][1] = fsqrt(fmad(R(0.25), q1, q2));
  g[2][2] = R(0.5) * fsqrt(fmad(r.x, r.x, q1));
}

// Diagonal majorisation of the rotational geometric stiffness
// (kernel.cuh:283-301).  For float, 0.5*x - y in float equals the reference's
// double evaluation rounded to float (no double rounding can occur).
// The 3x3 matrix is symmetric (its off-diagonal entries are bitwise equal:
// IEEE + and * commute), so six entries are formed; column sums keep row order.
template <class R> DUCK_HD void geometricAdd(Hess<R> &H, V3<R> r, V3<R> f) {
  R rf = fdot(r, f);
  R a00 = fmad(R(0.5), r.x * f.x + f.x * r.x, -rf);
  R a11 = fmad(R(0.5), r.y * f.y + f.y * r.y, -rf);
  R a22 = fmad(R(0.5), r.z * f.z + f.z * r.z, -rf);
  R a01 = R(0.5) * fmad(r.x, f.y, f.x * r.y);
  R a02 = R(0.5) * fmad(r.x, f.z, f.x * r.z);
  R a12 = R(0.5) * fmad(r.y, f.z, f.y * r.z);
  // (0 + a^2) is a^2: a square is never -0.
  H.h[tri(3, 3)] += fsqrt(fmad(a02, a02, fmad(a01, a01, a00 * a00)));
  H.h[tri(4, 4)] += fsqrt(fmad(a12, a12, fmad(a11, a11, a01 * a01)));
  H.h[tri(5, 5)] += fsqrt(fmad(a22, a22, fmad(a12, a12, a02 * a02)));
}

// Cholesky solve of H x = -g with NaN on a bad pivot (kernel.cuh:177-228).
// The float path multiplies by reciprocal pivots (fdivInv).  The factor runs
// to the end without branching; a non-positive or non-finite pivot anywhere
// replaces the whole solution by NaN, as the reference's early return does.
// The float path factors H = L D L^T instead (the same pivots d = l^2, so the
// same failure test, without the square roots on the pivot chain).
template <class R> DUCK_HD void solve6(const Hess<R> &H, R x[6]) {
  if constexpr (sizeof(R) == sizeof(float)) {
    R W[21], U[21], invD[6]; // W = L D (below the diagonal), U = L
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
#pragma unroll
      for (int j = 0; j <= i; ++j) {
        R v = H.h[tri(i, j)];
#pragma unroll
        for (int k = 0; k < j; ++k)
          v = fmad(-W[tri(i, k)], U[tri(j, k)], v);
        if (i == j) {
          ok = ok && v > 0 && mfinite(v);
          invD[i] = frcp(v);
        } else {
          W[tri(i, j)] = v;
          U[tri(i, j)] = v * invD[j];
        }
      }
    }
    R y[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      y[i] = -H.g[i];
#pragma unroll
      for (int k = 0; k < i; ++k)
        y[i] = fmad(-U[tri(i, k)], y[k], y[i]);
    }
#pragma unroll
    for (int i = 5; i >= 0; --i) {
      x[i] = y[i] * invD[i];
#pragma unroll
      for (int k = i + 1; k < 6; ++k)
        x[i] = fmad(-U[tri(k, i)], x[k], x[i]);
    }
#pragma unroll
    for (int k = 0; k < 6; ++k)
      x[k] = ok ? x[k] : R(NAN);
    return;
  }
  R L[21], inv[6];
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 6; ++i) {
#pragma unroll
    for (int j = 0; j <= i; ++j) {
      R v = H.h[tri(i, j)];
#pragma unroll
      for (int k = 0; k < j; ++k)
        v = fmad(-L[tri(i, k)], L[tri(j, k)], v);
      if (i == j) {
        ok = ok && v > 0 && mfinite(v);
        L[tri(i, i)] = fsqrt(v);
        inv[i] = frcp(L[tri(i, i)]);
      } else {
        L[tri(i, j)] = fdivInv(v, L[tri(j, j)], inv[j]);
      }
    }
  }
  R y[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    y[i] = -H.g[i];
#pragma unroll
    for (int k = 0; k < i; ++k)
      y[i] = fmad(-L[tri(i, k)], y[k], y[i]);
    y[i] = fdivInv(y[i], L[tri(i, i)], inv[i]);
  }
#pragma unroll
  for (int i = 5; i >= 0; --i) {
    x[i] = y[i];
#pragma unroll
    for (int k = i + 1; k < 6; ++k)
      x[i] = fmad(-L[tri(k, i)], x[k], x[i]);
    x[i] = fdivInv(x[i], L[tri(i, i)], inv[i]);
  }
#pragma unroll
  for (int k = 0; k < 6; ++k)
    x[k] = ok ? x[k] : R(NAN);
}

// (1 - (a/2)/tan(a/2)) / a^2, the SO(3) log-Jacobian coefficient, evaluated
// in double as the reference's float build does (kernel.cuh:841-850). [double]
// The float solver sums the series 1/12 + a^2/720 + a^4/30240 + a^6/1209600
// + a^8/47900160 for a < 0.5 (first omitted term < 1e-11 relative).
template <class R> DUCK_HD R logJacobianCoef(R a) {
  if constexpr (sizeof(R) == sizeof(float)) {
    if (a < R(0.5)) {
      R a2 = a * a;
      return fmad(a2, fmad(a2, fmad(a2, fmad(a2, R(1.0 / 47900160), R(1.0 / 1209600)), R(1.0 / 30240)),
                           R(1.0 / 720)),
                  R(1.0 / 12));
    }
  }
  double ad = double(a);
  if (ad < 1e-5)
    return R(1.0 / 12 + double(a * a / R(720)));
  return R((1 - 0.5 * ad / tan(0.5 * ad)) / double(a * a));
}

template <class R> DUCK_HD V3<R> unitAxis(int k) {
  return V3<R>{k == 0 ? R(1) : R(0), k == 1 ? R(1) : R(0), k == 2 ? R(1) : R(0)};
}

// The rotational Jacobian columns e_k - (theta x e_k) / 2 + coef theta x
// (theta x e_k) (kernel.cuh:851-858) with the unit axes' zeros dropped:
// theta x (theta x e_k) = theta theta_k - e_k |theta|^2.  The float solver's
// form (a reordering of the reference's sums).
template <class R> DUCK_HD void rotationJacobianSparse(V3<R> t, R coef, V3<R> rotJ[3]) {
  const R xy = coef * (t.x * t.y), xz = coef * (t.x * t.z), yz = coef * (t.y * t.z);
  const R xx = t.x * t.x, yy = t.y * t.y, zz = t.z * t.z;
  rotJ[0] = {fmad(-coef, yy + zz, R(1)), fmad(R(-0.5), t.z, xy), fmad(R(0.5), t.y, xz)};
  rotJ[1] = {fmad(R(0.5), t.z, xy), fmad(-coef, xx + zz, R(1)), fmad(R(-0.5), t.x, yz)};
  rotJ[2] = {fmad(R(-0.5), t.y, xz), fmad(R(0.5), t.x, yz), fmad(-coef, xx + yy, R(1))};
}

// Coulomb-projected contact force (kernel.cuh:304-315).
template <class R> DUCK_HD V3<R> contactForce(V3<R> C, const R lambda[3], const R penalty[3],
                                              R friction) {
  V3<R> f{fmad(penalty[0], C.x, lambda[0]), fmad(penalty[1], C.y, lambda[1]),
          fmad(penalty[2], C.z, lambda[2])};
  f.z = mn(f.z, R(0));
  R t = fhypot(f.x, f.y), bound = -friction * f.z;
  // the cone projection, selected rather than branched around
  const bool cap = t > bound && t > 0;
  const R ratio = fdiv(bound, t);
  f.x = cap ? f.x * ratio : f.x;
  f.y = cap ? f.y * ratio : f.y;
  return f;
}

// Value of the lane 8 positions away inside the same 16-lane row (DPP
// row_ror:8, i.e. lane ^ 8): the two halves of a split block solve.  A row
// rotation reads an in-range lane for every lane, so bound_ctrl (zero for
// out-of-range sources) changes nothing; it lets the compiler fold the move
// into the add that consumes it (v_add_f32_dpp).
__device__ __forceinline__ float pairSwap(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, true));
}
__device__ __forceinline__ double pairSwap(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const unsigned lo = __builtin_amdgcn_update_dpp(0, int(unsigned(b)), 0x128, 0xF, 0xF, true);
  const unsigned hi = __builtin_amdgcn_update_dpp(0, int(unsigned(b >> 32)), 0x128, 0xF, 0xF, true);
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}
// Value of lane ^ 16 (ds_swizzle, 32-lane groups: and 0x1f, xor 0x10).
__device__ __forceinline__ float halfSwap(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ double halfSwap(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const unsigned lo = __builtin_amdgcn_ds_swizzle(int(unsigned(b)), 0x401F);
  const unsigned hi = __builtin_amdgcn_ds_swizzle(int(unsigned(b >> 32)), 0x401F);
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// R diag(I) R^T of the body inertia at orientation q, as its six entries
// (xx, yy, zz, xy, xz, yz), and the product of such a matrix with v.
template <class R> DUCK_HD void inertiaWorld(Q4<R> q, V3<R> I, R out[6]) {
  V3<R> c0 = frotate(q, V3<R>{1, 0, 0}), c1 = frotate(q, V3<R>{0, 1, 0}),
        c2 = frotate(q, V3<R>{0, 0, 1}); // columns of R
  auto entry = [&](R a0, R a1, R a2, R b0, R b1, R b2) {
    return fmad(a2 * I.z, b2, fmad(a1 * I.y, b1, a0 * I.x * b0));
  };
  out[0] = entry(c0.x, c1.x, c2.x, c0.x, c1.x, c2.x);
  out[1] = entry(c0.y, c1.y, c2.y, c0.y, c1.y, c2.y);
  out[2] = entry(c0.z, c1.z, c2.z, c0.z, c1.z, c2.z);
  out[3] = entry(c0.x, c1.x, c2.x, c0.y, c1.y, c2.y);
  out[4] = entry(c0.x, c1.x, c2.x, c0.z, c1.z, c2.z);
  out[5] = entry(c0.y, c1.y, c2.y, c0.z, c1.z, c2.z);
}
template <class R> DUCK_HD V3<R> symApply(const R m[6], V3<R> v) {
  return {fmad(m[4], v.z, fmad(m[3], v.y, m[0] * v.x)), fmad(m[5], v.z, fmad(m[1], v.y, m[3] * v.x)),
          fmad(m[2], v.z, fmad(m[5], v.y, m[4] * v.x))};
}

// Lane (i - N) mod 16 of the same 16-lane row (DPP row_ror:N).
template <int N> __device__ __forceinline__ float rowRotate(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, true));
}
template <int N> __device__ __forceinline__ double rowRotate(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const unsigned lo = __builtin_amdgcn_update_dpp(0, int(unsigned(b)), 0x120 + N, 0xF, 0xF, true);
  const unsigned hi = __builtin_amdgcn_update_dpp(0, int(unsigned(b >> 32)), 0x120 + N, 0xF, 0xF, true);
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Lanes per block solve by default: one with up to 8 lanes per
// environment, two with 16, four with 32.
constexpr int defaultSolveLanes(int L) { return L >= 32 ? 4 : (L >= 16 ? 2 : 1); }

// Pairs: the model may have body-body contacts (without them, the rows and
// the two-pass assembly of body contacts are left out).
template <class R, int B, int J, int CG, int CS, int L, int PL = defaultSolveLanes(L), bool Pairs = true>
struct Stepper {
  using Env = EnvLds<R, B, J, CG, CS, L>;
  using Fr = Frames<R, B, J>;
  const DeviceModel<R> &M;
  const V3<R> *points;
  const Fr &F;
  Env &E;
  int lane; // 0..L-1 within the environment
  // Lanes per block solve: one (the reference's accumulation order), or
  // with 16 lanes per environment two lanes (lane, lane ^ 8), with 32 lanes
  // four (lane ^ 8, ^ 16, ^ 24) that share each body's assembly and sum it by
  // DPP row rotation / swizzle.
  static constexpr int P = PL;
  static_assert(P == 1 || (P == 2 && L == 16) || (P == 4 && L == 32),
                "split block solves: two lanes with 16 per environment, four with 32");
  // 64-bit words of a body's ground-contact mask
  static constexpr int GW = (CG + 63) / 64;

  // Ground contacts of body bi.
  __device__ int groundCount(int bi) const {
    int n = 0;
#pragma unroll
    for (int w = 0; w < GW; ++w)
      n += __popcll(E.gmask[w][bi]);
    return n;
  }
  // Index of body bi's n-th ground contact (from 0, list order), or -1.
  __device__ int nthGround(int bi, int n) const {
#pragma unroll
    for (int w = 0; w < GW; ++w) {
      uint64_t m = E.gmask[w][bi];
      const int c = __popcll(m);
      if (n < c) {
        for (int k = 0; k < n; ++k)
          m &= m - 1;
        return 64 * w + __builtin_ctzll(m);
      }
      n -= c;
    }
    return -1;
  }

  // ------------------------------------------------------------ access --
  DUCK_HD V3<R> X(int b) const { return {E.s.x[0][b], E.s.x[1][b], E.s.x[2][b]}; }
  DUCK_HD Q4<R> Q(int b) const { return {E.s.q[0][b], E.s.q[1][b], E.s.q[2][b], E.s.q[3][b]}; }
  DUCK_HD V3<R> Vel(int b) const { return {E.s.v[0][b], E.s.v[1][b], E.s.v[2][b]}; }
  DUCK_HD V3<R> Omega(int b) const { return {E.s.w[0][b], E.s.w[1][b], E.s.w[2][b]}; }
  DUCK_HD V3<R> Inertia(int b) const {
    return {E.s.inertia[0][b], E.s.inertia[1][b], E.s.inertia[2][b]};
  }
  DUCK_HD Q4<R> Q0(int b) const { return {E.q0[0][b], E.q0[1][b], E.q0[2][b], E.q0[3][b]}; }
  DUCK_HD void setX(int b, V3<R> v) {
    E.s.x[0][b] = v.x;
    E.s.x[1][b] = v.y;
    E.s.x[2][b] = v.z;
  }
  DUCK_HD void setQ(int b, Q4<R> q) {
    E.s.q[0][b] = q.w;
    E.s.q[1][b] = q.x;
    E.s.q[2][b] = q.y;
    E.s.q[3][b] = q.z;
  }
  DUCK_HD V3<R> frame(const R (&a)[3][J], int j) const { return {a[0][j], a[1][j], a[2][j]}; }
  DUCK_HD R forceZ(int b) const { return b == 1 ? E.s.force[2] : R(0); }
  DUCK_HD V3<R> force(int b) const {
    return b == 1 ? V3<R>{E.s.force[0], E.s.force[1], E.s.force[2]} : V3<R>{0, 0, 0};
  }
  // Inertia frozen at q0 (kernel.cuh:275-280).
  DUCK_HD V3<R> inertiaApply(Q4<R> q0, V3<R> I, V3<R> w, bool inverse) const {
    V3<R> l = frotate(conj(q0), w);
    if (inverse) {
      l.x *= R(1) / I.x;
      l.y *= R(1) / I.y;
      l.z *= R(1) / I.z;
    } else {
      l.x *= I.x;
      l.y *= I.y;
      l.z *= I.z;
    }
    return frotate(q0, l);
  }
  DUCK_HD R groundFriction(int shape) const {
    const R own = E.s.friction, model = F.shapeFriction[shape];
    return own >= 0 ? own : model;
  }

  // Hinge constraint values (kernel.cuh:732-761): anchor (3), axis (2),
  // limits (2); also returns the world frames used by the Jacobians.
  struct JointEval {
    R C[7], angle;
    V3<R> ra, rb, axis, axisB, t1, t2;
  };
  DUCK_HD JointEval evalJoint(int ji) const { return evalJoint(ji, F.a[ji], F.b[ji]); }
  DUCK_HD JointEval evalJoint(int ji, int a, int b) const {
    JointEval o;
    Q4<R> qa = Q(a), qb = Q(b);
    V3<R> u;
    if constexpr (sizeof(R) == sizeof(float)) {
      // Six frame vectors by two rotation matrices (the float solver).
      R ma[9], mb[9];
      quatMatrix(qa, ma);
      quatMatrix(qb, mb);
      o.ra = matApply(ma, frame(F.ra, ji));
      o.axis = matApply(ma, frame(F.axisA, ji));
      o.t1 = matApply(ma, frame(F.tangentA, ji));
      o.rb = matApply(mb, frame(F.rb, ji));
      o.axisB = matApply(mb, frame(F.axisB, ji));
      u = matApply(mb, frame(F.tangentB, ji));
    } else {
      o.ra = frotate(qa, frame(F.ra, ji));
      o.rb = frotate(qb, frame(F.rb, ji));
      o.axis = frotate(qa, frame(F.axisA, ji));
      o.axisB = frotate(qb, frame(F.axisB, ji));
      o.t1 = frotate(qa, frame(F.tangentA, ji));
      u = frotate(qb, frame(F.tangentB, ji));
    }
    V3<R> d = ((X(a) + o.ra) - X(b)) - o.rb;
    o.t2 = fcross(o.axis, o.t1);
    o.angle = fatan2(fdot(o.axis, fcross(o.t1, u)), fdot(o.t1, u));
    o.C[0] = d.x;
    o.C[1] = d.y;
    o.C[2] = d.z;
    o.C[3] = fdot(o.t1, o.axisB);
    o.C[4] = fdot(o.t2, o.axisB);
    o.C[5] = o.angle - F.lo[ji];
    o.C[6] = F.hi[ji] - o.angle;
    return o;
  }

  // Ground contact values in the fixed world basis (kernel.cuh:805-827).
  DUCK_HD V3<R> groundC(const GroundContact<R> &c, V3<R> &ra) const {
    int b = gcBody(c.id);
    ra = frotate(Q(b), V3<R>{c.local[0], c.local[1], c.local[2]});
    V3<R> delta = (X(b) + ra) - V3<R>{c.anchor[0], c.anchor[1], R(0)};
    delta.z = fmad(-M.alpha, c.c0, delta.z);
    return delta;
  }
  DUCK_HD V3<R> selfC(const SelfContact<R> &c, V3<R> &ra, V3<R> &rb) const {
    int a = scBody(c.id), b = scOther(c.id);
    ra = frotate(Q(a), V3<R>{c.local[0], c.local[1], c.local[2]});
    rb = frotate(Q(b), V3<R>{c.localB[0], c.localB[1], c.localB[2]});
    V3<R> delta = ((X(a) + ra) - X(b)) - rb;
    V3<R> t1{c.t1[0], c.t1[1], c.t1[2]}, t2{c.t2[0], c.t2[1], c.t2[2]}, n{c.n[0], c.n[1], c.n[2]};
    V3<R> C{fdot(delta, t1), fdot(delta, t2), fdot(delta, n)};
    C.z = fmad(-M.alpha, c.c0, C.z);
    return C;
  }

  // ----------------------------------------------------- dual updates --
  // New multipliers and penalties of hinge ji (kernel.cuh:991-1028) and the
  // hinge's terms folded into the iteration's error, from loads only; the
  // caller stores them after computing its other items, so that loads and
  // arithmetic of independent items form one block.  With valid false the
  // hinge geometry is evaluated for hinge 0 and the result is slot ji's own
  // values unchanged (ji < J: an unused slot), so the store needs no branch;
  // the error is left as it was.
  struct JointDual {
    R lambda[7], penalty[7], lambdaF, penaltyF;
    // inputs of the dry-friction part, kept for frictionDual
    R errRows, angle, fl, lambdaF0, penaltyF0;
    bool rough, wide;
    R C[5]; // anchor and axis constraint values (the step's diagnostics)
    JointEval je; // the evaluation (the next first pass may reuse it)
  };
  // Dry-friction multiplier and penalty of a hinge for the wrapped angle
  // change `delta`; returns the error after the hinge's terms.
  __device__ R frictionDual(JointDual &o, R delta) const {
    const R trial = fmad(o.penaltyF0, delta, o.lambdaF0);
    const R ramped = mn(fmad(M.betaAngular, mabs(delta), o.penaltyF0), R(1e7));
    o.lambdaF = o.rough ? clampv(trial, -o.fl, o.fl) : o.lambdaF0;
    o.penaltyF = (o.rough & (mabs(trial) < o.fl)) ? ramped : o.penaltyF0;
    const R residual = fmad(o.penaltyF, delta, o.lambdaF);
    const R fErr = mx(o.errRows, fdiv(mabs(o.lambdaF - clampv(residual, -o.fl, o.fl)), o.penaltyF));
    return o.rough ? fErr : o.errRows;
  }
  // The angle change is wrapped by wrapAngle's |a| < 3.14159 form (a + 0);
  // `wide` marks a lane outside it, which the caller completes with
  // frictionDual(o, wrapAngle(o.angle)) -- a branch kept out of this block.
  // `ends` is F.a[jg] | F.b[jg] << 8 (jg = valid ? ji : 0), which a lane may
  // hold in a register for its first hinge.
  __device__ JointDual jointDual(int ji, bool valid, R &error, int ends) const {
    const int jg = valid ? ji : 0;
    const R alpha = M.alpha;
    const JointEval je = evalJoint(jg, ends & 255, ends >> 8);
    JointDual o;
    o.je = je;
    R err = error;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      const R c = fmad(-alpha, E.c0[k][jg], je.C[k]);
      const R pen = E.s.penalty[k][ji], lam = E.s.lambda[k][ji];
      o.lambda[k] = valid ? fmad(pen, c, lam) : lam;
      const R ramped = mn(fmad(k < 3 ? M.betaLinear : M.betaAngular, mabs(c), pen), k < 3 ? R(1e9) : R(1e7));
      o.penalty[k] = valid ? ramped : pen;
      err = mx(err, mabs(c));
    }
    const bool limited = valid & (F.limited[jg] != 0);
#pragma unroll
    for (int k = 5; k < 7; ++k) {
      const R c = fmad(-alpha, mn(E.c0[k][jg], R(0)), je.C[k]);
      const R pen = E.s.penalty[k][ji], lam = E.s.lambda[k][ji];
      const R f = fmad(pen, c, lam);
      o.lambda[k] = limited ? mn(f, R(0)) : lam;
      const R ramped = mn(fmad(M.betaAngular, mabs(c), pen), R(1e7));
      o.penalty[k] = (limited & (f < 0)) ? ramped : pen;
      err = limited ? mx(err, mx(R(0), -c)) : err;
    }
    o.errRows = err;
#pragma unroll
    for (int k = 0; k < 5; ++k)
      o.C[k] = je.C[k];
    o.angle = je.angle - E.angle0[jg];
    o.fl = E.s.frictionloss[jg];
    o.lambdaF0 = E.s.lambdaF[ji];
    o.penaltyF0 = E.s.penaltyF[ji];
    o.rough = valid & (o.fl > 0);
    o.wide = valid & !(mabs(o.angle) < R(3.14159));
    err = frictionDual(o, o.angle + R(0));
    error = valid ? err : error;
    return o;
  }
  __device__ void storeJointDual(int ji, const JointDual &o) {
#pragma unroll
    for (int k = 0; k < 7; ++k) {
      E.s.lambda[k][ji] = o.lambda[k];
      E.s.penalty[k][ji] = o.penalty[k];
    }
    E.s.lambdaF[ji] = o.lambdaF;
    E.s.penaltyF[ji] = o.penaltyF;
  }
  // New force, penalties and stick flag of ground contact i (kernel.cuh:
  // 1029-1052), as jointDual does for a hinge (with valid false: slot i's
  // own values, i < CG, geometry from body 0).
  struct GroundDual {
    int id;
    R lambda[3], penalty[3];
    R depth; // max(0, -z) of the contact point (the step's diagnostics)
  };
  // `owner` is the contact's body | shape << 8 (0 when not valid), which a
  // lane may hold in a register for its first contact (fixed within a step).
  __device__ GroundDual groundDual(int i, bool valid, R &error, int owner) const {
    const GroundContact<R> &c = E.s.gc[i];
    const int id = c.id;
    const int b = owner & 255, shape = owner >> 8;
    const V3<R> ra = frotate(Q(b), V3<R>{c.local[0], c.local[1], c.local[2]});
    V3<R> C = (X(b) + ra) - V3<R>{c.anchor[0], c.anchor[1], R(0)};
    C.z = fmad(-M.alpha, c.c0, C.z);
    const R mu = groundFriction(shape);
    const R lam[3] = {c.lambda[0], c.lambda[1], c.lambda[2]}, pen[3] = {c.penalty[0], c.penalty[1], c.penalty[2]};
    const V3<R> f = contactForce(C, lam, pen, mu);
    const R trial = fhypot(fmad(pen[0], C.x, lam[0]), fmad(pen[1], C.y, lam[1]));
    const R slip = fhypot(C.x, C.y);
    const bool stick = trial <= -mu * f.z && double(slip) < 1e-5;
    GroundDual o;
    o.depth = mx(R(0), -(C.z + M.alpha * c.c0));
    const int idNew = (id & 0x7fffffff) | (stick ? int(0x80000000u) : 0);
    const R errNew = mx(error, mx(R(0), -C.z));
    o.id = valid ? idNew : id;
    const R fk[3] = {f.x, f.y, f.z}, Ck[3] = {C.x, C.y, C.z};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      o.lambda[k] = valid ? fk[k] : lam[k];
      const bool ramp = valid & (f.z < 0) & ((k == 2) | (trial <= -mu * f.z));
      const R ramped = mn(fmad(M.betaLinear, mabs(Ck[k]), pen[k]), R(1e9));
      o.penalty[k] = ramp ? ramped : pen[k];
    }
    error = valid ? errNew : error;
    return o;
  }
  __device__ void storeGroundDual(int i, const GroundDual &o) {
    GroundContact<R> &c = E.s.gc[i];
    c.id = o.id;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      c.lambda[k] = o.lambda[k];
      c.penalty[k] = o.penalty[k];
    }
  }

  // --------------------------------------------------- 6x6 block solve --
  // kernel.cuh:828-936 for one dynamic body.  With P > 1 the P lanes of a
  // group call this for the same body: part 0 assembles the inertia block,
  // and the i-th hinge and the n-th contact of the body go to part
  // (i + 1) mod P and (n + 1) mod P; the partial systems are summed on every
  // lane of the group (bitwise the same sum: the pairwise sums commute), all
  // factor, part 0 writes the pose.
  // Inertia block (kernel.cuh:837-855), assigned into the zeroed H (the
  // first terms of every sum).  With P >= 2 the first two lanes share it:
  // both form theta, the log-Jacobian and rotJ; part 0 applies the world
  // inertia to theta and rotJ[0] (the g rows and the first rotational
  // column, plus the linear block), part 1 to rotJ[1] and rotJ[2] (the other
  // three rotational entries); further parts add nothing.
  // Fast (float): straight-line, on the small-rotation branches of flogmap
  // and logJacobianCoef only -- bitwise their results there -- with `slow`
  // set where a lane's rotation lies outside them.
  template <bool Fast> __device__ void inertiaBlock(Hess<R> &H, int bi, int part, bool &slow) const {
    const R h = M.dt, h2 = h * h, ih2 = frcp(h2);
    const V3<R> x = X(bi), xp{E.xp[0][bi], E.xp[1][bi], E.xp[2][bi]};
    const Q4<R> q = Q(bi), qp{E.qp[0][bi], E.qp[1][bi], E.qp[2][bi], E.qp[3][bi]};
    if (!Fast && part >= 2)
      return;
    V3<R> theta;
    R coef;
    if constexpr (Fast) {
      // flogmap: normalise, fold to w >= 0, 2 atan(s/w)/s by its series.
      Q4<R> d = fqmul(q, conj(qp));
      const R n2 = fmad(d.z, d.z, fmad(d.y, d.y, fmad(d.x, d.x, d.w * d.w)));
      const R inv = frsqrt(n2);
      const R sg = d.w * inv < 0 ? R(-1) : R(1);
      d = {(d.w * inv) * sg, (d.x * inv) * sg, (d.y * inv) * sg, (d.z * inv) * sg};
      const V3<R> v{d.x, d.y, d.z};
      const R sv = fnorm(v);
      const R iw = frcp(d.w), t = sv * iw, t2 = t * t;
      const R series =
          fmad(t2, fmad(t2, fmad(t2, fmad(t2, fmad(t2, R(-1.0 / 11), R(1.0 / 9)), R(-1.0 / 7)), R(0.2)),
                        R(-1.0 / 3)),
               R(1));
      const R k = double(sv) < 1e-10 ? R(2) : (R(2) * iw) * series;
      theta = v * k;
      const R a = fnorm(theta), a2 = a * a;
      coef = fmad(a2, fmad(a2, fmad(a2, fmad(a2, R(1.0 / 47900160), R(1.0 / 1209600)), R(1.0 / 30240)),
                           R(1.0 / 720)),
                  R(1.0 / 12));
      slow = slow | (double(n2) < 1e-30) | !(d.w > R(0.99)) | !(a < R(0.5));
    } else {
      theta = flogmap(fqmul(q, conj(qp)));
      coef = logJacobianCoef(fnorm(theta));
    }
    V3<R> rotJ[3];
    if constexpr (Fast) {
      rotationJacobianSparse(theta, coef, rotJ);
    } else {
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        V3<R> e = unitAxis<R>(k);
        rotJ[k] = faxpy(coef, fcross(theta, fcross(theta, e)), faxpy(R(-0.5), fcross(theta, e), e));
      }
    }
    // World inertia at q0, formed once per step by the predictor.
    const R Iw[6] = {E.Iw[0][bi], E.Iw[1][bi], E.Iw[2][bi], E.Iw[3][bi], E.Iw[4][bi], E.Iw[5][bi]};
    const bool first = part == 0, second = part == 1;
    const V3<R> dx = x - xp;
    const R mh = fdivInv(E.s.mass[bi], h2, ih2);
    H.h[tri(0, 0)] = first ? mh : R(0);
    H.h[tri(1, 1)] = first ? mh : R(0);
    H.h[tri(2, 2)] = first ? mh : R(0);
    H.g[0] = first ? mh * dx.x : R(0);
    H.g[1] = first ? mh * dx.y : R(0);
    H.g[2] = first ? mh * dx.z : R(0);
    if constexpr (P == 1) {
      V3<R> It = symApply(Iw, theta);
      V3<R> IJ[3] = {symApply(Iw, rotJ[0]), symApply(Iw, rotJ[1]), symApply(Iw, rotJ[2])};
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        H.g[3 + k] = fdivInv(fdot(rotJ[k], It), h2, ih2);
#pragma unroll
        for (int l = 0; l <= k; ++l)
          H.h[tri(3 + k, 3 + l)] = fdivInv(fdot(rotJ[k], IJ[l]), h2, ih2);
      }
    } else {
      const V3<R> A = symApply(Iw, first ? theta : rotJ[1]);
      const V3<R> Bv = symApply(Iw, first ? rotJ[0] : rotJ[2]);
      const R d0 = fdivInv(fdot(rotJ[0], A), h2, ih2), d1 = fdivInv(fdot(rotJ[1], A), h2, ih2),
              d2 = fdivInv(fdot(rotJ[2], A), h2, ih2);
      const R e0 = fdivInv(fdot(rotJ[0], Bv), h2, ih2), e1 = fdivInv(fdot(rotJ[1], Bv), h2, ih2),
              e2 = fdivInv(fdot(rotJ[2], Bv), h2, ih2);
      H.g[3] = first ? d0 : R(0);
      H.g[4] = first ? d1 : R(0);
      H.g[5] = first ? d2 : R(0);
      H.h[tri(3, 3)] = first ? e0 : R(0);
      H.h[tri(4, 3)] = first ? e1 : R(0);
      H.h[tri(5, 3)] = first ? e2 : R(0);
      H.h[tri(4, 4)] = second ? d1 : R(0);
      H.h[tri(5, 4)] = second ? d2 : R(0);
      H.h[tri(5, 5)] = second ? e2 : R(0);
    }
  }

  // Rows of one hinge adjacent to body bi (kernel.cuh:861-913); `cur` packs
  // (hinge, body a, body b).  With valid false the rows are stamped with zero
  // force and stiffness on hinge 0's geometry between world bodies (finite:
  // the staged frames of absent hinges are zero), so the same straight-line
  // code serves a lane without a hinge in this slot.
  // Fast: both wrapped angles on wrapAngle's |a| < 3.14159 branch, `slow`
  // set otherwise; the two limit rows and the axis rows, all along +-J5, are
  // one stamp with the summed force and stiffness (float sums reordered).
  // Given: `given` is this hinge's evaluation at the current poses, made by
  // the dual update (evalJoint is not repeated).
  template <bool Fast, bool Given = false>
  __device__ void hingeRows(Hess<R> &H, int bi, int cur, bool valid, bool implicitDrive,
                            bool &slow, const JointEval *given = nullptr) const {
    const R h = M.dt, h2 = h * h, ih2 = frcp(h2), ih = frcp(h), alpha = M.alpha;
    const int ji = valid ? cur & 255 : 0, ja = valid ? (cur >> 8) & 255 : 0,
              jb = valid ? (cur >> 16) & 255 : 0;
    const bool parent = bi == ja;
    const R s = parent ? R(1) : R(-1);
    JointEval je;
    if constexpr (Given)
      je = *given;
    else
      je = evalJoint(ji, ja, jb);
    if (!Fast && !valid)
      return;
    // Anchor rows (k = 0..2): J_k = [s e_k, r x e_k] with r = ra (parent)
    // or -rb (child); their geometric terms share r.  Anchor and axis rows
    // are always active; the limit rows on limited hinges with f < 0 (the
    // rest are stamped with zeros, which adds nothing).
    const V3<R> r = parent ? je.ra : -je.rb;
    R geo[3][3];
    axisGeometricNorms(r, geo);
    R fr[5], pr[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      // loads first, selects after: a conditional load would be a branch
      const R c = fmad(-alpha, E.c0[k][ji], je.C[k]);
      const R pen = E.s.penalty[k][ji], lam = E.s.lambda[k][ji];
      pr[k] = valid ? pen : R(0);
      fr[k] = valid ? fmad(pen, c, lam) : R(0);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      stampAxisRow(H, k, s, r, fr[k], pr[k]);
      const R af = mabs(fr[k]);
      H.h[tri(3, 3)] = fmad(af, geo[k][0], H.h[tri(3, 3)]);
      H.h[tri(4, 4)] = fmad(af, geo[k][1], H.h[tri(4, 4)]);
      H.h[tri(5, 5)] = fmad(af, geo[k][2], H.h[tri(5, 5)]);
    }
#pragma unroll
    for (int k = 3; k < 5; ++k) {
      const V3<R> t = k == 3 ? je.t1 : je.t2;
      if constexpr (Fast) {
        // The child's row is the parent's negated, (t x axisB) with -f, and
        // the geometric term is symmetric in its two vectors: no selects.
        stampAngular(H, fcross(t, je.axisB), s * fr[k], pr[k]);
        geometricAdd(H, t, je.axisB * fr[k]);
      } else {
        const V3<R> u = parent ? t : je.axisB, w = parent ? je.axisB : t;
        stampAngular(H, fcross(u, w), fr[k], pr[k]);
        geometricAdd(H, u, w * fr[k]);
      }
    }
    // Rows along the hinge axis (kernel.cuh:893-913): implicit torque-
    // limited PD potential, damping/armature, dry friction -- one stamp
    // with the summed force and stiffness, selected without branches.  The
    // lower limit row's Jacobian is J5, the upper's -J5.
    const V3<R> J5 = parent ? -je.axis : je.axis;
    const int lim = F.limited[ji];
    const bool limited = valid & (lim != 0);
    R limF[2], limK[2];
#pragma unroll
    for (int k = 5; k < 7; ++k) {
      const R c = fmad(-alpha, mn(E.c0[k][ji], R(0)), je.C[k]);
      const R pen = E.s.penalty[k][ji];
      const R f = mn(fmad(pen, c, E.s.lambda[k][ji]), R(0));
      const bool on = limited && f < 0;
      limF[k - 5] = on ? f : R(0);
      limK[k - 5] = on ? pen : R(0);
      if constexpr (!Fast)
        stampAngular(H, k == 5 ? J5 : -J5, limF[k - 5], limK[k - 5]);
    }
    R wTarget, delta;
    const R a0 = je.angle - E.s.target[ji], a1 = je.angle - E.angle0[ji];
    if constexpr (Fast) {
      wTarget = a0 + R(0);
      delta = a1 + R(0);
      slow = slow | (valid & !((mabs(a0) < R(3.14159)) & (mabs(a1) < R(3.14159))));
    } else {
      wrapAngle2(a0, a1, wTarget, delta);
    }
    const R kp = E.s.kp[ji], maxT = E.s.maxTorque[ji];
    R drive = fmad(kp, wTarget, -E.s.torque[ji]);
    const bool capped = maxT > 0;
    const R ks = capped && mabs(drive) >= maxT ? R(0) : kp;
    drive = capped ? clampv(drive, -maxT, maxT) : drive;
    R axisForce = implicitDrive ? drive : R(0), axisStiff = implicitDrive ? ks : R(0);
    const R damping = E.s.damping[ji], armature = F.armature[ji], w0 = E.velocity0[ji];
    const R dh = fdivInv(damping, h, ih), ah = fdivInv(armature, h2, ih2);
    const R stiff = dh + ah;
    const bool damped = stiff > 0;
    axisForce += damped ? fmad(dh, delta, ah * fmad(-h, w0, delta)) : R(0);
    axisStiff += damped ? stiff : R(0);
    const R fl = E.s.frictionloss[ji];
    const R trial = fmad(E.s.penaltyF[ji], delta, E.s.lambdaF[ji]);
    axisForce += fl > 0 ? clampv(trial, -fl, fl) : R(0);
    axisStiff += fl > 0 && mabs(trial) < fl ? E.s.penaltyF[ji] : R(0);
    if constexpr (Fast) {
      axisForce += limF[0] - limF[1];
      axisStiff += limK[0] + limK[1];
    }
    if constexpr (Fast) // J5 = -s axis: the stamp along axis with the force's sign flipped
      stampAngular(H, je.axis, valid ? -s * axisForce : R(0), valid ? axisStiff : R(0));
    else
      stampAngular(H, J5, valid ? axisForce : R(0), valid ? axisStiff : R(0));
  }

  // Rows of ground contact `index` of body bi (kernel.cuh:915-931).  A
  // separating contact (f.z = 0) is stamped with zero force and stiffness;
  // with valid false the lever arm is zero as well (index clamped in range).
  __device__ void groundRows(Hess<R> &H, int bi, int index, bool valid) const {
    const GroundContact<R> &c = E.s.gc[valid ? index : 0];
    const int id = c.id;
    V3<R> ra = frotate(Q(bi), V3<R>{c.local[0], c.local[1], c.local[2]});
    V3<R> C = (X(bi) + ra) - V3<R>{c.anchor[0], c.anchor[1], R(0)};
    C.z = fmad(-M.alpha, c.c0, C.z);
    V3<R> f = contactForce(C, c.lambda, c.penalty, groundFriction(valid ? gcShape(id) : 0));
    const bool on = valid && f.z < 0;
    if (!on)
      f = V3<R>{0, 0, 0};
    if (!valid)
      ra = V3<R>{0, 0, 0};
    stampAxisRow(H, 0, R(1), ra, f.x, on ? c.penalty[0] : R(0));
    stampAxisRow(H, 1, R(1), ra, f.y, on ? c.penalty[1] : R(0));
    stampAxisRow(H, 2, R(1), ra, f.z, on ? c.penalty[2] : R(0));
    geometricAdd(H, ra, f);
  }

  // Rows of body-body contact `index` touching body bi (kernel.cuh:915-931).
  __device__ void selfRows(Hess<R> &H, int bi, int index) const {
    const SelfContact<R> &c = E.s.sc[index];
    V3<R> ra, rb;
    V3<R> C = selfC(c, ra, rb);
    bool first = bi == scBody(c.id);
    V3<R> r = first ? ra : rb;
    R sign = first ? R(1) : R(-1);
    V3<R> f = contactForce(C, c.lambda, c.penalty, c.friction);
    if (f.z < 0) {
      V3<R> basis[3] = {{c.t1[0], c.t1[1], c.t1[2]}, {c.t2[0], c.t2[1], c.t2[2]}, {c.n[0], c.n[1], c.n[2]}};
      R fk[3] = {f.x, f.y, f.z};
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        V3<R> e = basis[k] * sign;
        stampFull(H, e, fcross(r, e), fk[k], c.penalty[k]);
      }
      V3<R> fw = ((basis[0] * f.x) + (basis[1] * f.y)) + (basis[2] * f.z);
      geometricAdd(H, r, fw * sign);
    }
  }

  // The assembly of one lane's share of body bi's system, in the reference's
  // order (inertia, hinges in adjacency order, ground contacts, body-body
  // contacts in list order).  The i-th hinge and the n-th contact of the
  // body go to part (i + 1) mod nParts and (n + 1) mod nParts.
  __device__ void assembleGeneric(Hess<R> &H, int bi, bool implicitDrive, int part, int nParts) const {
    bool slow = false;
#pragma unroll
    for (int k = 0; k < 21; ++k)
      H.h[k] = 0;
#pragma unroll
    for (int k = 0; k < 6; ++k)
      H.g[k] = 0;
    inertiaBlock<false>(H, bi, part, slow);
    // The next adjacency entry is fetched while the current hinge is stamped.
    const int adjEnd = F.adjStart[bi + 1];
    int adj = F.adjStart[bi] + (part + nParts - 1) % nParts;
    int packed = adj < adjEnd ? F.adj[adj] : 0;
    for (; adj < adjEnd; adj += nParts) {
      const int cur = packed;
      if (adj + nParts < adjEnd)
        packed = F.adj[adj + nParts];
      hingeRows<false>(H, bi, cur, true, implicitDrive, slow);
    }
    int nth = 0;
#pragma unroll
    for (int w = 0; w < GW; ++w)
      for (uint64_t m = E.gmask[w][bi]; m; m &= m - 1, ++nth)
        if ((nth + 1) % nParts == part % nParts)
          groundRows(H, bi, 64 * w + __builtin_ctzll(m), true);
    nth = 0;
    for (uint32_t m = Pairs ? E.smask[bi] : 0u; m; m &= m - 1, ++nth)
      if ((nth + 1) % nParts == part % nParts)
        selfRows(H, bi, __builtin_ctz(m));
  }

  // The float assembly: the inertia block, the lane's first hinge and (with
  // Ground) its first two ground contacts as one straight-line block --
  // independent chains the scheduler interleaves -- then any further hinges
  // and contacts by the generic loops.  Contacts are added before further
  // hinges (a reordering of the sums, float only).  Returns false when a
  // lane's rotation or angle left the fast forms' range.
  // What the float assembly of body bi on one lane reads before its first
  // hinge and contacts: the lane's first hinge (packed), its first two
  // ground contacts (positions p0 and p0 + nParts among the body's) and the
  // range of its further hinges.  Model adjacency and the step's contact
  // masks only, so fixed for a whole step: a lane computes it once per step
  // for its bodies of the first two colours and keeps the two words in
  // registers, and the assembly starts on the hinge data without the
  // dependent adjacency loads.
  struct SlotPlan {
    int w0; // first hinge (hinge | a << 8 | b << 16) | h0 << 24 | v0 << 25 | v1 << 26 | any contact << 27 | staged << 28
    int w1; // c0 | c1 << 8 | next hinge slot << 16 | end of the body's hinges << 24
  };
  __device__ SlotPlan plan(int bi, int part, int nParts) const {
    const int p0 = (part + nParts - 1) % nParts;
    const int adjEnd = F.adjStart[bi + 1], adj0 = F.adjStart[bi] + p0;
    const bool h0 = adj0 < adjEnd;
    const int packed0 = F.adj[h0 ? adj0 : 0];
    bool v0, v1, any;
    int c0, c1;
    if constexpr (GW == 1) {
      const uint64_t all = E.gmask[0][bi];
      uint64_t m = all;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        m = k < p0 ? m & (m - 1) : m;
      v0 = m != 0;
      c0 = v0 ? __builtin_ctzll(m) : 0;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        m = k < nParts ? m & (m - 1) : m;
      v1 = m != 0;
      c1 = v1 ? __builtin_ctzll(m) : 0;
      any = all != 0;
    } else {
      c0 = nthGround(bi, p0);
      c1 = nthGround(bi, p0 + nParts);
      v0 = c0 >= 0;
      v1 = c1 >= 0;
      c0 = v0 ? c0 : 0;
      c1 = v1 ? c1 : 0;
      any = groundCount(bi) != 0;
    }
    return {packed0 | int(h0) << 24 | int(v0) << 25 | int(v1) << 26 | int(any) << 27,
            c0 | c1 << 8 | (adj0 + nParts) << 16 | adjEnd << 24};
  }

  template <bool Ground, bool Given>
  __device__ bool assembleFast(Hess<R> &H, int bi, bool implicitDrive, int part, int nParts,
                               SlotPlan sp, const JointEval *given) const {
    bool slow = false;
#pragma unroll
    for (int k = 0; k < 21; ++k)
      H.h[k] = 0;
#pragma unroll
    for (int k = 0; k < 6; ++k)
      H.g[k] = 0;
    const int p0 = (part + nParts - 1) % nParts;
    const int packed0 = sp.w0 & 0xffffff;
    const bool h0 = (sp.w0 >> 24) & 1;
    const int adjNext = (sp.w1 >> 16) & 255, adjEnd = (sp.w1 >> 24) & 255;
    inertiaBlock<true>(H, bi, part, slow);
    hingeRows<true, Given>(H, bi, packed0, h0, implicitDrive, slow, given);
    if constexpr (Ground) {
      groundRows(H, bi, sp.w1 & 255, (sp.w0 >> 25) & 1);
      groundRows(H, bi, (sp.w1 >> 8) & 255, (sp.w0 >> 26) & 1);
    }
    for (int adj = adjNext; adj < adjEnd; adj += nParts)
      hingeRows<true>(H, bi, F.adj[adj], true, implicitDrive, slow);
    if constexpr (GW == 1) {
      // The lane's further contacts (positions p0 + k nParts beyond the
      // straight-line ones), one per lane per round, the rounds counted by a
      // ballot: the lanes of a wave stamp their k-th further contact together
      // (a round without one stamps zeros).  Each lane adds the same contacts
      // in the same order as a walk over the body's list.
      uint64_t m = E.gmask[0][bi];
      if constexpr (Ground) {
        // the contacts after the lane's second straight-line one, then the
        // other parts' nParts - 1
        const int c1 = (sp.w1 >> 8) & 255;
        m = (sp.w0 >> 26) & 1 ? m & ~((2ull << c1) - 1) : 0ull;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          m = k < nParts - 1 ? m & (m - 1) : m;
      } else {
#pragma unroll
        for (int k = 0; k < 3; ++k)
          m = k < p0 ? m & (m - 1) : m;
      }
      while (__any(m != 0)) {
        const bool v = m != 0;
        groundRows(H, bi, v ? __builtin_ctzll(m) : 0, v);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          m = k < nParts ? m & (m - 1) : m;
      }
    } else {
      int nth = 0;
#pragma unroll
      for (int w = 0; w < GW; ++w)
        for (uint64_t g = E.gmask[w][bi]; g; g &= g - 1, ++nth)
          if ((!Ground || nth >= 2 * nParts) && nth % nParts == p0)
            groundRows(H, bi, 64 * w + __builtin_ctzll(g), true);
    }
    int nth = 0;
    for (uint32_t g = Pairs ? E.smask[bi] : 0u; g; g &= g - 1, ++nth)
      if (nth % nParts == p0)
        selfRows(H, bi, __builtin_ctz(g));
    return !slow;
  }

  // --------------------------------------------------- 6x6 block solve --
  // kernel.cuh:828-936 for one dynamic body.  With P > 1 the P lanes of a
  // group call this for the same body, each assembling its share; the
  // partial systems are summed on every lane of the group (bitwise the same
  // sum: the pairwise sums commute), all factor, part 0 writes the pose.
  // nParts (<= 4) is the size of this body's lane group when a colour pass
  // gives one body two slots (slots 0 and 4, lane and lane ^ 8 in each), and
  // `quad` tells every lane of the wave that such a group exists in this pass.
  // `sp` is plan(bi, part, nParts) (float only).  Given: `given` is the
  // evaluation of the lane's first hinge at the current poses (float only).
  // A body solved alone in a later colour may be assembled in two passes:
  // a lane whose plan has bit 28 of its first word set (float only; the
  // body's smask word is zero then) assembles its share of every row but the
  // body contacts into E.staged[part] and leaves the pose alone (returning
  // 0); a lane with `finish` set starts from that share and adds the
  // body-contact rows of E.earlyMask -- the same sums in the same order as
  // one assembly.
  template <bool Given = false>
  __device__ R updateBody(int bi, bool implicitDrive, int part, int nParts, bool quad, SlotPlan sp,
                          const JointEval *given = nullptr, bool finish = false) {
    const bool stage = Pairs && sizeof(R) == sizeof(float) && ((sp.w0 >> 28) & 1);
    const V3<R> x = X(bi);
    const Q4<R> q = Q(bi);
    Hess<R> H;
    if (Pairs && finish) {
#pragma unroll
      for (int k = 0; k < 21; ++k)
        H.h[k] = E.staged[part][k];
#pragma unroll
      for (int k = 0; k < 6; ++k)
        H.g[k] = E.staged[part][21 + k];
      const int p0 = (part + nParts - 1) % nParts;
      int nth = 0;
      for (uint32_t g = E.earlyMask; g; g &= g - 1, ++nth)
        if (nth % nParts == p0)
          selfRows(H, bi, __builtin_ctz(g));
    } else {
      bool done = false;
      if constexpr (sizeof(R) == sizeof(float)) {
        // Wave-uniform choices: with or without the straight-line contacts,
        // and the generic assembly for every lane when any lane fell outside
        // the fast forms.
        const bool fast =
            __any((sp.w0 >> 27) & 1)
                ? assembleFast<true, Given>(H, bi, implicitDrive, part, nParts, sp, given)
                : assembleFast<false, Given>(H, bi, implicitDrive, part, nParts, sp, given);
        done = !__any(!fast);
      }
      if (!done)
        assembleGeneric(H, bi, implicitDrive, part, nParts);
      if (stage) {
#pragma unroll
        for (int k = 0; k < 21; ++k)
          E.staged[part][k] = H.h[k];
#pragma unroll
        for (int k = 0; k < 6; ++k)
          E.staged[part][21 + k] = H.g[k];
      }
    }
    if constexpr (P >= 2) {
#pragma unroll
      for (int k = 0; k < 21; ++k)
        H.h[k] += pairSwap(H.h[k]);
#pragma unroll
      for (int k = 0; k < 6; ++k)
        H.g[k] += pairSwap(H.g[k]);
    }
    if constexpr (P == 4) {
#pragma unroll
      for (int k = 0; k < 21; ++k)
        H.h[k] += halfSwap(H.h[k]);
#pragma unroll
      for (int k = 0; k < 6; ++k)
        H.g[k] += halfSwap(H.g[k]);
    } else if constexpr (P == 2) {
      if (quad) {
        // A two-slot group (slots 0 and 4 of the row: lanes 0, 8 and 4, 12)
        // adds the other slot's pair sum, which lane i finds in lane i - 12
        // (mod 16) in both slots.  Both then hold (a + b) + (c + d) and
        // (c + d) + (a + b): bitwise equal.
        const bool four = nParts == 4;
#pragma unroll
        for (int k = 0; k < 21; ++k) {
          const R o = H.h[k] + rowRotate<12>(H.h[k]);
          H.h[k] = four ? o : H.h[k];
        }
#pragma unroll
        for (int k = 0; k < 6; ++k) {
          const R o = H.g[k] + rowRotate<12>(H.g[k]);
          H.g[k] = four ? o : H.g[k];
        }
      }
    }
    R st[6];
    solve6(H, st);
    V3<R> tx{st[0], st[1], st[2]}, rx{st[3], st[4], st[5]};
    const R ntx = fnorm(tx), nrx = fnorm(rx);
    R scale = mn(R(1), mn(fdiv(R(.1), mx(ntx, R(1e-30))), fdiv(R(.25), mx(nrx, R(1e-30)))));
    if (part == 0 && !stage) {
      setX(bi, faxpy(scale, tx, x));
      setQ(bi, fnormalized(fqmul(fexpmap(scale * rx), q)));
    }
    return stage ? R(0) : mx(ntx, nrx) * scale;
  }
};

} // namespace duckhip
