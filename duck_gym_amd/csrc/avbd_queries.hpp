// Per-environment kernels that read or initialise the HBM state directly
// (one lane per environment): initialise, masked reset, state snapshot and
// the contact/load queries of the reference batch (src/cuda/extension.cu:
// 22-50, 128-159, 175-185).
#pragma once
#include "avbd_kernels.hpp"

namespace duckhip {

template <class R, int B, int J, int CG, int CS> struct StateView {
  using State = EnvState<R, B, J, CG, CS>;
  const DeviceModel<R> &M;
  State &s;
  DUCK_HD V3<R> X(int b) const { return {s.x[0][b], s.x[1][b], s.x[2][b]}; }
  DUCK_HD Q4<R> Q(int b) const { return {s.q[0][b], s.q[1][b], s.q[2][b], s.q[3][b]}; }
  DUCK_HD V3<R> W(int b) const { return {s.w[0][b], s.w[1][b], s.w[2][b]}; }
  DUCK_HD V3<R> mv(const R (&a)[3][kMaxModelJoints], int j) const { return {a[0][j], a[1][j], a[2][j]}; }
  DUCK_HD R angle(int j) const {
    return hingeAngle(Q(M.ja[j]), Q(M.jb[j]), mv(M.axisA, j), mv(M.tangentA, j), mv(M.tangentB, j));
  }
  DUCK_HD void setX(int b, V3<R> v) {
    s.x[0][b] = v.x;
    s.x[1][b] = v.y;
    s.x[2][b] = v.z;
  }
  DUCK_HD void setQ(int b, Q4<R> q) {
    s.q[0][b] = q.w;
    s.q[1][b] = q.x;
    s.q[2][b] = q.y;
    s.q[3][b] = q.z;
  }
  // Copy of the model state (kernel.cuh:383-396).
  DUCK_HD void initialize() {
    for (int b = 0; b < M.nb; ++b) {
      for (int k = 0; k < 3; ++k) {
        s.x[k][b] = M.x[k][b];
        s.v[k][b] = M.v[k][b];
        s.w[k][b] = M.w[k][b];
        s.inertia[k][b] = M.inertia[k][b];
      }
      for (int k = 0; k < 4; ++k)
        s.q[k][b] = M.q[k][b];
      s.mass[b] = M.mass[b];
    }
    for (int k = 0; k < 3; ++k)
      s.force[k] = 0;
    for (int j = 0; j < M.nj; ++j) {
      for (int k = 0; k < 7; ++k) {
        s.lambda[k][j] = 0;
        s.penalty[k][j] = k < 3 ? R(1000) : R(1);
      }
      s.lambdaF[j] = 0;
      s.penaltyF[j] = 1;
      s.target[j] = M.target[j];
      s.kp[j] = M.kp[j];
      s.maxTorque[j] = M.maxTorque[j];
      s.torque[j] = M.torque[j];
      s.frictionloss[j] = M.frictionloss[j];
      s.damping[j] = M.damping[j];
    }
    for (int k = 0; k < 8; ++k)
      s.diag[k] = 0;
    s.friction = -1;
    s.colorCount = 2;
    for (int b = 0; b < B; ++b)
      s.colors[b] = b < M.nb ? M.colors[b] : 0;
    s.modelColours = 1;
    s.drive = kDriveOther;
    s.failed = 0;
    s.ngc = 0;
    s.nsc = 0;
  }
  // Clears the claims of `drive` and `modelColours` that the blob's bytes do
  // not bear out (an imported state); keeps every true one, so that an export
  // and import of the same batch's state is the identity.
  DUCK_HD void checkStamps() {
    bool ok = true;
    if (s.drive == kDriveTarget || s.drive == kDriveMotor) {
      const bool target = s.drive == kDriveTarget;
      for (int j = 0; j < J; ++j) {
        const bool in = j < M.nj;
        ok = ok && sameBits(s.kp[j], in && target ? s.driveKp : R(0)) &&
             sameBits(s.maxTorque[j], in && target ? s.driveLimit : R(0));
        if (target)
          ok = ok && sameBits(s.torque[j], in ? M.torque[j] : R(0)) &&
               sameBits(s.frictionloss[j], in ? M.frictionloss[j] : R(0)) &&
               sameBits(s.damping[j], in ? M.damping[j] : R(0));
      }
    } else {
      ok = s.drive == kDriveOther;
    }
    if (!ok)
      s.drive = kDriveOther;
    if (s.modelColours != 0) {
      bool same = s.modelColours == 1;
      for (int b = 0; b < B; ++b)
        same = same && s.colors[b] == (b < M.nb ? M.colors[b] : 0);
      if (!same)
        s.modelColours = 0;
    }
  }
  // Root offset and forward kinematics down the hinge list (kernel.cuh:397-420).
  DUCK_HD void resetPose(const R *q, const R *root) {
    for (int b = 0; b < M.nb; ++b)
      for (int k = 0; k < 3; ++k) {
        s.v[k][b] = 0;
        s.w[k][b] = 0;
      }
    for (int k = 0; k < 3; ++k)
      s.force[k] = 0;
    setX(1, X(1) + V3<R>{root[0], root[1], root[2]});
    setQ(1, expmap(V3<R>{root[3], root[4], root[5]}) * Q(1));
    for (int j = 0; j < M.nj; ++j) {
      const int a = M.ja[j], b = M.jb[j];
      Q4<R> oa{M.q[0][a], M.q[1][a], M.q[2][a], M.q[3][a]};
      Q4<R> ob{M.q[0][b], M.q[1][b], M.q[2][b], M.q[3][b]};
      Q4<R> qa = Q(a);
      V3<R> axis = rotate(qa, mv(M.axisA, j));
      Q4<R> qb = normalized(((expmap(axis * (q[j] - M.originalAngle[j])) * qa) * conj(oa)) * ob);
      setQ(b, qb);
      setX(b, (X(a) + rotate(qa, mv(M.ra, j))) - rotate(qb, mv(M.rb, j)));
    }
  }
};

template <class R, int B, int J, int CG, int CS>
__global__ void initializeKernel(const DeviceModel<R> *model, unsigned char *states,
                                 long long blobBytes, int count) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  StateView<R, B, J, CG, CS> v{*model, blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e)};
  v.initialize();
}

template <class R, int B, int J, int CG, int CS>
__global__ void checkStampsKernel(const DeviceModel<R> *model, unsigned char *states,
                                  long long blobBytes, int count) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  StateView<R, B, J, CG, CS> v{*model, blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e)};
  v.checkStamps();
}

// ext (optional, per env): [friction (<0 keeps the shape friction),
// mass scale, vx, vy, vz] -- batch extensions with no reference counterpart.
template <class R, int B, int J, int CG, int CS>
__global__ void resetKernel(const DeviceModel<R> *model, unsigned char *states, long long blobBytes,
                            int count, const unsigned char *mask, const R *q, const R *root,
                            const R *ext) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count || !mask[e])
    return;
  const DeviceModel<R> &M = *model;
  auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  const R *qe = q + size_t(e) * M.nj, *re = root + size_t(e) * 6;
  for (int k = 0; k < 6; ++k)
    if (!mfinite(re[k])) {
      s.failed = 1;
      return;
    }
  for (int k = 0; k < M.nj; ++k)
    if (!mfinite(qe[k])) {
      s.failed = 1;
      return;
    }
  if (ext)
    for (int k = 0; k < 5; ++k)
      if (!mfinite(ext[size_t(e) * 5 + k])) {
        s.failed = 1;
        return;
      }
  StateView<R, B, J, CG, CS> v{M, s};
  v.initialize();
  v.resetPose(qe, re);
  if (ext) {
    const R *x = ext + size_t(e) * 5;
    s.friction = x[0];
    for (int b = 0; b < M.nb; ++b)
      if (s.mass[b] > 0) {
        s.mass[b] *= x[1];
        for (int k = 0; k < 3; ++k) {
          s.inertia[k][b] *= x[1];
          s.v[k][b] = x[2 + k];
        }
      }
  }
}

// bodies [E,B,13], joints [E,J,2], diag [E,6] (kernel.cuh:555-575).
template <class R, int B, int J, int CG, int CS>
__global__ void snapshotKernel(const DeviceModel<R> *model, unsigned char *states,
                               long long blobBytes, int count, R *bodies, R *joints, R *diag) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  const DeviceModel<R> &M = *model;
  auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  StateView<R, B, J, CG, CS> v{M, s};
  R *bo = bodies + size_t(e) * M.nb * 13;
  for (int b = 0; b < M.nb; ++b) {
    R row[13] = {s.x[0][b], s.x[1][b], s.x[2][b], s.q[0][b], s.q[1][b], s.q[2][b], s.q[3][b],
                 s.v[0][b], s.v[1][b], s.v[2][b], s.w[0][b], s.w[1][b], s.w[2][b]};
    for (int k = 0; k < 13; ++k)
      bo[13 * b + k] = row[k];
  }
  R *jo = joints + size_t(e) * M.nj * 2;
  for (int j = 0; j < M.nj; ++j) {
    jo[2 * j] = v.angle(j);
    jo[2 * j + 1] = dot(v.W(M.jb[j]) - v.W(M.ja[j]), rotate(v.Q(M.ja[j]), v.mv(M.axisA, j)));
  }
  R *d = diag + size_t(e) * 6;
  d[0] = s.diag[kJointError];
  d[1] = s.diag[kPenetration];
  d[2] = s.diag[kContacts];
  d[3] = s.diag[kConverged];
  d[4] = s.diag[kAxisError];
  d[5] = R(s.failed);
}

template <class R> DUCK_HD V3<R> selfForceWorld(const SelfContact<R> &c) {
  return ((V3<R>{c.t1[0], c.t1[1], c.t1[2]} * c.lambda[0]) +
          (V3<R>{c.t2[0], c.t2[1], c.t2[2]} * c.lambda[1])) +
         (V3<R>{c.n[0], c.n[1], c.n[2]} * c.lambda[2]);
}

// The z component of contactForcesKernel's row for body b (ground and body
// contacts): the same terms summed in the same order.
template <class R, int B, int J, int CG, int CS>
DUCK_HD R contactForceZ(const EnvState<R, B, J, CG, CS> &s, int b) {
  R z = 0;
  for (int i = 0; i < s.ngc; ++i) {
    const auto &c = s.gc[i];
    const V3<R> f = -((V3<R>{1, 0, 0} * c.lambda[0] + V3<R>{0, 1, 0} * c.lambda[1]) +
                      V3<R>{0, 0, 1} * c.lambda[2]);
    if (gcBody(c.id) == b)
      z += f.z;
  }
  for (int i = 0; i < s.nsc; ++i) {
    const auto &c = s.sc[i];
    const V3<R> f = -selfForceWorld(c);
    if (scBody(c.id) == b)
      z += f.z;
    if (scOther(c.id) == b)
      z -= f.z;
  }
  return z;
}

// [E,B,3] contact force on each body (kernel.cuh:467-480).
template <class R, int B, int J, int CG, int CS>
__global__ void contactForcesKernel(const DeviceModel<R> *model, unsigned char *states,
                                    long long blobBytes, int count, int groundOnly, R *out) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  const DeviceModel<R> &M = *model;
  auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  R *o = out + size_t(e) * M.nb * 3;
  for (int i = 0; i < M.nb * 3; ++i)
    o[i] = 0;
  for (int i = 0; i < s.ngc; ++i) {
    const auto &c = s.gc[i];
    // contactWorld with the fixed basis, negated.
    V3<R> f = -((V3<R>{1, 0, 0} * c.lambda[0] + V3<R>{0, 1, 0} * c.lambda[1]) +
                V3<R>{0, 0, 1} * c.lambda[2]);
    int b = gcBody(c.id);
    o[b * 3] += f.x;
    o[b * 3 + 1] += f.y;
    o[b * 3 + 2] += f.z;
  }
  if (groundOnly)
    return;
  for (int i = 0; i < s.nsc; ++i) {
    const auto &c = s.sc[i];
    V3<R> f = -selfForceWorld(c);
    int a = scBody(c.id), b = scOther(c.id);
    o[a * 3] += f.x;
    o[a * 3 + 1] += f.y;
    o[a * 3 + 2] += f.z;
    o[b * 3] -= f.x;
    o[b * 3 + 1] -= f.y;
    o[b * 3 + 2] -= f.z;
  }
}

// [E,2] active body-body contacts and maximum depth (kernel.cuh:481-493).
template <class R, int B, int J, int CG, int CS>
__global__ void selfContactStatsKernel(const DeviceModel<R> *model, unsigned char *states,
                                       long long blobBytes, int count, R *out) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  const DeviceModel<R> &M = *model;
  auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  StateView<R, B, J, CG, CS> v{M, s};
  R n = 0, depthMax = 0;
  for (int i = 0; i < s.nsc; ++i) {
    const auto &c = s.sc[i];
    int a = scBody(c.id), b = scOther(c.id);
    V3<R> ra = rotate(v.Q(a), V3<R>{c.local[0], c.local[1], c.local[2]});
    V3<R> rb = rotate(v.Q(b), V3<R>{c.localB[0], c.localB[1], c.localB[2]});
    V3<R> delta = ((v.X(a) + ra) - v.X(b)) - rb;
    R cz = dot(delta, V3<R>{c.n[0], c.n[1], c.n[2]}) - M.alpha * c.c0;
    R depth = mx(R(0), -(cz + M.alpha * c.c0));
    if (c.lambda[2] < R(-1e-5) || depth > R(1e-6))
      n += 1;
    depthMax = mx(depthMax, depth);
  }
  out[2 * e] = n;
  out[2 * e + 1] = depthMax;
}

template <class R, int B, int J, int CG, int CS>
__global__ void contactCountsKernel(unsigned char *states, long long blobBytes, int count, R *out) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  out[2 * e] = R(s.ngc);
  out[2 * e + 1] = R(s.nsc);
}

// The per-body quantities of the Newton-Euler pass.
template <class R, int B> struct RneaWork {
  V3<R> acc[B], alpha[B], force[B], moment[B], contact[B], contactMoment[B];
};

// Recursive Newton-Euler at zero joint acceleration (kernel.cuh:504-554):
// per hinge [bias, contact/limit, applied actuator torque] into o[3 j + k];
// `off` is the root COM offset of the acceleration reference point.  `work`
// holds the per-body quantities (private memory, or a caller's LDS scratch).
template <class R, int B, int J, int CG, int CS>
DUCK_HD void rneaLoadsIn(const DeviceModel<R> &M, const EnvState<R, B, J, CG, CS> &s, const R *off,
                         R *o, RneaWork<R, B> &work) {
  StateView<R, B, J, CG, CS> v{M, const_cast<EnvState<R, B, J, CG, CS> &>(s)};
  V3<R> *acc = work.acc, *alpha = work.alpha, *force = work.force, *moment = work.moment,
        *contact = work.contact, *contactMoment = work.contactMoment;
  for (int b = 0; b < M.nb; ++b)
    acc[b] = alpha[b] = force[b] = moment[b] = contact[b] = contactMoment[b] = V3<R>{0, 0, 0};
  acc[1] = cross(v.W(1), cross(v.W(1), rotate(v.Q(1), V3<R>{off[0], off[1], off[2]})));
  for (int j = 0; j < M.nj; ++j) {
    const int a = M.ja[j], b = M.jb[j];
    Q4<R> qa = v.Q(a), qb = v.Q(b);
    V3<R> axis = rotate(qa, v.mv(M.axisA, j)), ra = rotate(qa, v.mv(M.ra, j)),
          rb = rotate(qb, v.mv(M.rb, j));
    V3<R> wa = v.W(a), wb = v.W(b);
    R speed = dot(wb - wa, axis);
    alpha[b] = alpha[a] + cross(wa, axis) * speed;
    acc[b] = (((acc[a] + cross(alpha[a], ra)) + cross(wa, cross(wa, ra))) - cross(alpha[b], rb)) -
             cross(wb, cross(wb, rb));
  }
  for (int b = 1; b < M.nb; ++b) {
    Q4<R> q = v.Q(b);
    V3<R> I{s.inertia[0][b], s.inertia[1][b], s.inertia[2][b]}, w = v.W(b);
    auto inertia = [&](V3<R> u) {
      V3<R> l = rotate(conj(q), u);
      l.x *= I.x;
      l.y *= I.y;
      l.z *= I.z;
      return rotate(q, l);
    };
    force[b] = (acc[b] - V3<R>{M.gravity[0], M.gravity[1], M.gravity[2]}) * s.mass[b];
    moment[b] = inertia(alpha[b]) + cross(w, inertia(w));
  }
  for (int i = 0; i < s.ngc; ++i) {
    const auto &c = s.gc[i];
    V3<R> f = -((V3<R>{1, 0, 0} * c.lambda[0] + V3<R>{0, 1, 0} * c.lambda[1]) +
                V3<R>{0, 0, 1} * c.lambda[2]);
    int b = gcBody(c.id);
    contact[b] = contact[b] + f;
    contactMoment[b] =
        contactMoment[b] + cross(rotate(v.Q(b), V3<R>{c.local[0], c.local[1], c.local[2]}), f);
  }
  for (int i = 0; i < s.nsc; ++i) {
    const auto &c = s.sc[i];
    V3<R> f = -selfForceWorld(c);
    int a = scBody(c.id), b = scOther(c.id);
    contact[a] = contact[a] + f;
    contactMoment[a] =
        contactMoment[a] + cross(rotate(v.Q(a), V3<R>{c.local[0], c.local[1], c.local[2]}), f);
    contact[b] = contact[b] + (-f);
    contactMoment[b] = contactMoment[b] +
                       cross(rotate(v.Q(b), V3<R>{c.localB[0], c.localB[1], c.localB[2]}), -f);
  }
  for (int k = M.nj - 1; k >= 0; --k) {
    const int a = M.ja[k], b = M.jb[k];
    Q4<R> qa = v.Q(a), qb = v.Q(b);
    V3<R> axis = rotate(qa, v.mv(M.axisA, k)), rb = rotate(qb, v.mv(M.rb, k)),
          shift = v.X(b) - v.X(a);
    o[3 * k] = dot(axis, moment[b] - cross(rb, force[b]));
    o[3 * k + 1] = dot(axis, contactMoment[b] - cross(rb, contact[b])) +
                   (M.limited[k] ? -s.lambda[5][k] + s.lambda[6][k] : R(0));
    R motor = s.torque[k] - s.kp[k] * wrapAngle(v.angle(k) - s.target[k]);
    o[3 * k + 2] = s.maxTorque[k] > 0 ? clampv(motor, -s.maxTorque[k], s.maxTorque[k]) : motor;
    moment[a] = moment[a] + (moment[b] + cross(shift, force[b]));
    force[a] = force[a] + force[b];
    contactMoment[a] = contactMoment[a] + (contactMoment[b] + cross(shift, contact[b]));
    contact[a] = contact[a] + contact[b];
  }
}
template <class R, int B, int J, int CG, int CS>
DUCK_HD void rneaLoads(const DeviceModel<R> &M, const EnvState<R, B, J, CG, CS> &s, const R *off,
                       R *o) {
  RneaWork<R, B> work;
  rneaLoadsIn<R, B, J, CG, CS>(M, s, off, o, work);
}

template <class R, int B, int J, int CG, int CS>
__global__ void generalizedLoadsKernel(const DeviceModel<R> *model, unsigned char *states,
                                       long long blobBytes, int count, const R *offset, R *out) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  const auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  rneaLoads<R, B, J, CG, CS>(*model, s, offset + size_t(e) * 3, out + size_t(e) * model->nj * 3);
}

} // namespace duckhip
