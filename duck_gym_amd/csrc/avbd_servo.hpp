// Servo substep of the BAM-actuated environment (python/duck_gym/bam_env.py:
// 307-326 with the XL330/m6 equations of python/duck_gym/actuator.py:16-77):
// the delayed-target ring buffer, the external hinge load from a zero-
// acceleration Newton-Euler pass, and the motor model, producing the
// (torque, dry-friction budget, damping) channels the next implicit step
// consumes.  One lane per environment: the supply voltage couples the joints
// of an environment through sum |previous torque|.
#pragma once
#include "../../include/duck_hip.h"
#include "avbd_queries.hpp"

namespace duckhip {

DUCK_HD float mpow(float x, float y) { return powf(x, y); }
DUCK_HD double mpow(double x, double y) { return pow(x, y); }
DUCK_HD float mexpf(float x) { return expf(x); }
DUCK_HD double mexpf(double x) { return exp(x); }

// actuator.py:44-77 for one joint.  Scalar parameters are combined in the
// order torch evaluates them: a Python float meeting a tensor is rounded to
// the tensor dtype; products of Python floats are formed in double first.
template <class R>
DUCK_HD void xl330(const DuckServo &p, R supply, R target, R position, R velocity, R previousApplied,
                   R external, R &applied, R &budget, R &damping, R &raw) {
  R speed = velocity * R(p.kd_scale);
  const double errorGain = (4096 / (2 * 3.14159265358979323846)) / (256 * 885);
  R duty = (((target - position) * R(p.kp_fw)) * R(p.kp_scale)) * R(errorGain);
  R center = (R(p.kt) * speed) / supply;
  R span = R(p.resistance * 1.75) / supply;
  R lo = center - span, hi = center + span;
  duty = duty < lo ? lo : duty; // torch.clamp(min=lo, max=hi): min(max(x, lo), hi)
  duty = duty > hi ? hi : duty;
  duty = duty < R(-1) ? R(-1) : (duty > R(1) ? R(1) : duty);
  raw = ((R(p.kt) * supply) * duty) / R(p.resistance) - (R(p.kt * p.kt) * speed) / R(p.resistance);
  R stribeck = mexpf(-mpow(mabs(velocity) / R(p.dtheta_stribeck), R(p.alpha)));
  R mot = previousApplied, ext = external;
  R quad = mabs(mot) > mabs(ext) ? R(p.load_friction_external_quad) * (ext * ext)
                                 : R(p.load_friction_motor_quad) * (mot * mot);
  budget = ((((R(p.friction_base) + stribeck * R(p.friction_stribeck)) +
              mabs(ext * R(p.load_friction_external) - mot * R(p.load_friction_motor))) +
             stribeck * mabs(ext * R(p.load_friction_external_stribeck) -
                             mot * R(p.load_friction_motor_stribeck))) +
            stribeck * quad) *
           R(p.friction_scale);
  R limit = R(p.force_limit);
  applied = raw < -limit ? -limit : (raw > limit ? limit : raw);
  damping = R(p.friction_viscous);
}

struct ServoBuffers {
  const void *target;          // [E,J] commanded target of this control step
  void *history;               // [lag+1, E, J] ring buffer of targets
  int cursor;                  // slot written this substep
  unsigned char *initialized;  // [E] ring buffer filled since the last reset
  const void *rootOffset;      // [E,3] root COM offset for the load pass
  void *previousMotor;         // [E,J] raw motor torque of the last substep (in/out)
  void *previousApplied;       // [E,J] clamped torque of the last substep (in/out)
  void *motor;                 // [E,J,3] out
  void *supply;                // [E] out, may be null
};

template <class R, int B, int J, int CG, int CS>
__global__ void servoKernel(DuckServo p, const DeviceModel<R> *model, unsigned char *states,
                            long long blobBytes, int count, ServoBuffers io) {
  int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= count)
    return;
  const DeviceModel<R> &M = *model;
  const auto &s = blobAt<EnvState<R, B, J, CG, CS>>(states, blobBytes, e);
  StateView<R, B, J, CG, CS> view{M, const_cast<EnvState<R, B, J, CG, CS> &>(s)};
  const int nj = M.nj, slots = p.lag + 1;
  const size_t row = size_t(e) * nj, plane = size_t(count) * nj;
  const R *target = static_cast<const R *>(io.target) + row;
  R *history = static_cast<R *>(io.history);
  // bam_env.py:308-314: write this substep's target, fill a fresh ring, read
  // the target `lag` substeps old.
  for (int j = 0; j < nj; ++j)
    history[size_t(io.cursor) * plane + row + j] = target[j];
  if (!io.initialized[e]) {
    for (int k = 0; k < slots; ++k)
      for (int j = 0; j < nj; ++j)
        history[size_t(k) * plane + row + j] = target[j];
    io.initialized[e] = 1;
  }
  const int delayedSlot = ((io.cursor - p.lag) % slots + slots) % slots;
  const R *delayed = history + size_t(delayedSlot) * plane + row;

  R loads[J][3];
  rneaLoads<R, B, J, CG, CS>(M, s, static_cast<const R *>(io.rootOffset) + size_t(e) * 3,
                             &loads[0][0]);
  R *prevMotor = static_cast<R *>(io.previousMotor) + row;
  R *prevApplied = static_cast<R *>(io.previousApplied) + row;
  R total = 0;
  for (int j = 0; j < nj; ++j)
    total += mabs(prevMotor[j]);
  R supply = R(p.vin) - R(p.vin_drop_gain) * total;
  supply = supply < R(p.vin_min) ? R(p.vin_min) : supply;
  R *motor = static_cast<R *>(io.motor) + row * 3;
  for (int j = 0; j < nj; ++j) {
    R position = view.angle(j);
    R velocity = dot(view.W(M.jb[j]) - view.W(M.ja[j]), rotate(view.Q(M.ja[j]), view.mv(M.axisA, j)));
    R external = -loads[j][0] + loads[j][1];
    R applied, budget, damping, raw;
    xl330(p, supply, delayed[j], position, velocity, prevApplied[j], external, applied, budget,
          damping, raw);
    motor[3 * j] = applied;
    motor[3 * j + 1] = budget;
    motor[3 * j + 2] = damping;
    prevMotor[j] = raw;
    prevApplied[j] = applied;
  }
  if (io.supply)
    static_cast<R *>(io.supply)[e] = supply;
}

// rneaLoadsIn split over an environment's L lanes, for a model whose hinges
// form a tree listed parent first (M.jointLevels > 0): the outward pass one
// tree level at a time (a hinge reads only its parent body, final after the
// level before), the per-body forces and the contact sums one body per lane
// (a body's contacts in list order, ground then body contacts), the inward
// pass from the deepest level: each hinge of the level writes its loads, then
// each parent adds its children's terms in decreasing hinge order.  Every
// quantity is formed by the operations of rneaLoadsIn in its order, so the
// loads are bitwise those of the sequential pass.  Every lane of the
// workgroup calls it (barriers); `valid` lanes work.
template <class R, int B, int J, int CG, int CS, int L>
__device__ __forceinline__ void rneaLoadsLanes(const DeviceModel<R> &M,
                                               const EnvState<R, B, J, CG, CS> &s, const R *off,
                                               R *o, RneaWork<R, B> &work, int lane, bool valid) {
  constexpr int BPL = (B + L - 1) / L, JPL = (J + L - 1) / L;
  StateView<R, B, J, CG, CS> v{M, const_cast<EnvState<R, B, J, CG, CS> &>(s)};
  V3<R> *acc = work.acc, *alpha = work.alpha, *force = work.force, *moment = work.moment,
        *contact = work.contact, *contactMoment = work.contactMoment;
  const int nb = M.nb, nj = M.nj, levels = M.jointLevels;
  // the lane's hinges and bodies: level, ends, child hinges (read once); a
  // hinge's world axis and child arm, formed in the outward pass, serve the
  // inward pass too (the poses do not move in between); its actuator column
  // needs no tree quantity and is written first
  int jLevel[JPL], jA[JPL], jB[JPL], bLevel[BPL];
  unsigned children[BPL];
  V3<R> jAxis[JPL], jRb[JPL];
#pragma unroll
  for (int r = 0; r < JPL; ++r) {
    const int j = lane + r * L;
    const bool in = valid && j < nj;
    jLevel[r] = in ? M.jointLevel[j] : -1;
    jA[r] = in ? M.ja[j] : 0;
    jB[r] = in ? M.jb[j] : 0;
    jAxis[r] = jRb[r] = V3<R>{0, 0, 0};
    if (in) {
      R motor = s.torque[j] - s.kp[j] * wrapAngle(v.angle(j) - s.target[j]);
      o[3 * j + 2] = s.maxTorque[j] > 0 ? clampv(motor, -s.maxTorque[j], s.maxTorque[j]) : motor;
    }
  }
#pragma unroll
  for (int r = 0; r < BPL; ++r) {
    const int b = lane + r * L;
    const bool in = valid && b < nb;
    bLevel[r] = in ? M.bodyLevel[b] : -1;
    children[r] = in ? M.childHinges[b] : 0u;
    if (in)
      acc[b] = alpha[b] = force[b] = moment[b] = contact[b] = contactMoment[b] = V3<R>{0, 0, 0};
  }
  __syncthreads();
  if (valid && lane == 0)
    acc[1] = cross(v.W(1), cross(v.W(1), rotate(v.Q(1), V3<R>{off[0], off[1], off[2]})));
  __syncthreads();
  for (int level = 1; level <= levels; ++level) {
#pragma unroll
    for (int r = 0; r < JPL; ++r) {
      const int j = lane + r * L;
      if (jLevel[r] != level)
        continue;
      const int a = jA[r], b = jB[r];
      Q4<R> qa = v.Q(a), qb = v.Q(b);
      V3<R> axis = rotate(qa, v.mv(M.axisA, j)), ra = rotate(qa, v.mv(M.ra, j)),
            rb = rotate(qb, v.mv(M.rb, j));
      V3<R> wa = v.W(a), wb = v.W(b);
      R speed = dot(wb - wa, axis);
      alpha[b] = alpha[a] + cross(wa, axis) * speed;
      acc[b] = (((acc[a] + cross(alpha[a], ra)) + cross(wa, cross(wa, ra))) - cross(alpha[b], rb)) -
               cross(wb, cross(wb, rb));
      jAxis[r] = axis;
      jRb[r] = rb;
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < BPL; ++r) {
    const int b = lane + r * L;
    if (!valid || b < 1 || b >= nb)
      continue;
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
    V3<R> sum{0, 0, 0}, sumMoment{0, 0, 0};
    for (int i = 0; i < s.ngc; ++i) {
      const auto &c = s.gc[i];
      if (gcBody(c.id) != b)
        continue;
      V3<R> f = -((V3<R>{1, 0, 0} * c.lambda[0] + V3<R>{0, 1, 0} * c.lambda[1]) +
                  V3<R>{0, 0, 1} * c.lambda[2]);
      sum = sum + f;
      sumMoment = sumMoment + cross(rotate(q, V3<R>{c.local[0], c.local[1], c.local[2]}), f);
    }
    for (int i = 0; i < s.nsc; ++i) {
      const auto &c = s.sc[i];
      const int ca = scBody(c.id), cb = scOther(c.id);
      if (ca != b && cb != b)
        continue;
      V3<R> f = -selfForceWorld(c);
      if (ca == b) {
        sum = sum + f;
        sumMoment = sumMoment + cross(rotate(q, V3<R>{c.local[0], c.local[1], c.local[2]}), f);
      }
      if (cb == b) {
        sum = sum + (-f);
        sumMoment = sumMoment + cross(rotate(q, V3<R>{c.localB[0], c.localB[1], c.localB[2]}), -f);
      }
    }
    contact[b] = sum;
    contactMoment[b] = sumMoment;
  }
  __syncthreads();
  for (int level = levels; level >= 1; --level) {
#pragma unroll
    for (int r = 0; r < JPL; ++r) {
      const int k = lane + r * L;
      if (jLevel[r] != level)
        continue;
      const int b = jB[r];
      const V3<R> axis = jAxis[r], rb = jRb[r];
      o[3 * k] = dot(axis, moment[b] - cross(rb, force[b]));
      o[3 * k + 1] = dot(axis, contactMoment[b] - cross(rb, contact[b])) +
                     (M.limited[k] ? -s.lambda[5][k] + s.lambda[6][k] : R(0));
    }
    if (level == 1)
      break; // the roots' sums feed no hinge
#pragma unroll
    for (int r = 0; r < BPL; ++r) {
      const int p = lane + r * L;
      if (bLevel[r] != level - 1)
        continue;
      // the body's child hinges in decreasing order, as the sequential pass
      for (unsigned m = children[r]; m; m &= ~(1u << (31 - __builtin_clz(m)))) {
        const int k = 31 - __builtin_clz(m);
        const int b = M.jb[k];
        V3<R> shift = v.X(b) - v.X(p);
        moment[p] = moment[p] + (moment[b] + cross(shift, force[b]));
        force[p] = force[p] + force[b];
        contactMoment[p] = contactMoment[p] + (contactMoment[b] + cross(shift, contact[b]));
        contact[p] = contact[p] + contact[b];
      }
    }
    __syncthreads();
  }
}

// The servo substep inside the step launch (servoStepKernel): the operations
// of servoKernel on the state the launch staged in LDS, before the motor
// step.  Lanes take hinges; the environment's lanes run the load pass one
// tree level at a time (rneaLoadsLanes; for a model whose hinges are no tree
// listed parent first, the first lane runs it in hinge order), with its
// per-body quantities in the step's per-step scratch, which the step fills
// later; the first lane sums the supply in servoKernel's order.  The channels
// go into `ctl`, where the motor step takes them.
template <class R, int B, int J, int CG, int CS, int L, int JPL, class Env>
__device__ __forceinline__ void servoPrologue(const ServoArgs<R> &sv, const DeviceModel<R> &M, Env &E,
                                              int e, int lane, bool valid, int count,
                                              R (&ctl)[JPL][3]) {
  static_assert(sizeof(RneaWork<R, B>) <= sizeof(R) * 20 * B, "the load pass fits x0 .. Iw");
  static_assert(3 * J < 7 * J - 1, "loads and supply fit c0");
  const int nj = M.nj, slots = sv.p.lag + 1;
  const size_t row = size_t(e) * nj, plane = size_t(count) * nj;
  R *loads = &E.c0[0][0];
  R delayed[JPL];
  if (valid) {
    // bam_env.py:308-314: this substep's target into the ring (every slot
    // of a fresh ring), the target `lag` substeps old out
    const bool fresh = !sv.initialized[e];
    const int delayedSlot = ((sv.cursor - sv.p.lag) % slots + slots) % slots;
#pragma unroll
    for (int r = 0; r < JPL; ++r) {
      const int j = lane + r * L;
      delayed[r] = 0;
      if (j >= nj)
        continue;
      const R t = sv.target[row + j];
      sv.history[size_t(sv.cursor) * plane + row + j] = t;
      if (fresh)
        for (int k = 0; k < slots; ++k)
          sv.history[size_t(k) * plane + row + j] = t;
      delayed[r] = sv.history[size_t(delayedSlot) * plane + row + j];
    }
  }
  auto &work = *reinterpret_cast<RneaWork<R, B> *>(&E.x0[0][0]);
  if (M.jointLevels > 0)
    rneaLoadsLanes<R, B, J, CG, CS, L>(M, E.s, sv.rootOffset + size_t(e) * 3, loads, work, lane,
                                       valid);
  if (valid) {
    if (lane == 0) {
      if (M.jointLevels == 0)
        rneaLoadsIn<R, B, J, CG, CS>(M, E.s, sv.rootOffset + size_t(e) * 3, loads, work);
      R total = 0;
      for (int j = 0; j < nj; ++j)
        total += mabs(sv.previousMotor[row + j]);
      R supply = R(sv.p.vin) - R(sv.p.vin_drop_gain) * total;
      supply = supply < R(sv.p.vin_min) ? R(sv.p.vin_min) : supply;
      E.c0[6][J - 1] = supply;
      if (sv.supply)
        sv.supply[e] = supply;
      sv.initialized[e] = 1;
    }
  }
  __syncthreads();
  if (valid) {
    StateView<R, B, J, CG, CS> view{M, E.s};
    const R supply = E.c0[6][J - 1];
#pragma unroll
    for (int r = 0; r < JPL; ++r) {
      const int j = lane + r * L;
      if (j >= nj)
        continue;
      R position = view.angle(j);
      R velocity = dot(view.W(M.jb[j]) - view.W(M.ja[j]), rotate(view.Q(M.ja[j]), view.mv(M.axisA, j)));
      R external = -loads[3 * j] + loads[3 * j + 1];
      R applied, budget, damping, raw;
      xl330(sv.p, supply, delayed[r], position, velocity, sv.previousApplied[row + j], external,
            applied, budget, damping, raw);
      if (sv.motor) {
        sv.motor[(row + j) * 3] = applied;
        sv.motor[(row + j) * 3 + 1] = budget;
        sv.motor[(row + j) * 3 + 2] = damping;
      }
      sv.previousMotor[row + j] = raw;
      sv.previousApplied[row + j] = applied;
      ctl[r][0] = applied;
      ctl[r][1] = budget;
      ctl[r][2] = damping;
    }
  }
  __syncthreads(); // the load pass's scratch is the step's
}

// torch.maximum: NaN when either operand is NaN.
template <class R> DUCK_HD R maximumNan(R a, R b) { return a != a || b != b ? R(NAN) : (a > b ? a : b); }

// The end of the servo substep, on the environment's first lane after the
// motor step: self_contact_stats (selfContactStatsKernel's loop) folded into
// the running maxima (bam_env.py:333-335), then refresh() (bam_env.py:128-
// 155) on the new state: gravity and velocities in the root frame, the
// ground contact force on each foot (contactForcesKernel's sums), the foot
// sites, the mean-velocity filter (bam_env.py:343-345) and the air/contact
// timers.
template <class R, int B, int J, int CG, int CS, class Env>
__device__ __forceinline__ void servoEpilogue(const ServoArgs<R> &sv, const DeviceModel<R> &M, Env &E,
                                              int e) {
  auto &s = E.s;
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
  if (sv.selfContacts)
    sv.selfContacts[e] = maximumNan(sv.selfContacts[e], n);
  if (sv.selfPenetration)
    sv.selfPenetration[e] = maximumNan(sv.selfPenetration[e], depthMax);
  auto put = [](R *out, size_t i, V3<R> u) {
    if (out) {
      out[3 * i] = u.x;
      out[3 * i + 1] = u.y;
      out[3 * i + 2] = u.z;
    }
  };
  const Q4<R> q1 = v.Q(1), root = q1 * Q4<R>{sv.rootInv[0], sv.rootInv[1], sv.rootInv[2], sv.rootInv[3]};
  const V3<R> w1 = v.W(1), v1{s.v[0][1], s.v[1][1], s.v[2][1]};
  put(sv.gravity, e, rotate(conj(root), V3<R>{0, 0, -1}));
  put(sv.angularVelocity, e, rotate(conj(root), w1));
  const R *off = sv.rootOffset + size_t(e) * 3;
  const V3<R> rootR = -rotate(q1, V3<R>{off[0], off[1], off[2]});
  const V3<R> origin = v1 + cross(w1, rootR);
  put(sv.originVelocity, e, origin);
  put(sv.linearVelocity, e, rotate(conj(root), origin));
  if (sv.meanVelocity) {
    // mean_velocity_world.lerp_(origin, alpha) (bam_env.py:343-345) as
    // mean + alpha (origin - mean)
    R *m = sv.meanVelocity + size_t(e) * 3;
    m[0] = m[0] + sv.meanAlpha * (origin.x - m[0]);
    m[1] = m[1] + sv.meanAlpha * (origin.y - m[1]);
    m[2] = m[2] + sv.meanAlpha * (origin.z - m[2]);
  }
  const R h = M.dt;
  for (int f = 0; f < sv.numFeet; ++f) {
    const int body = sv.feet[f];
    const size_t k = size_t(e) * sv.numFeet + f;
    V3<R> force{0, 0, 0};
    for (int i = 0; i < s.ngc; ++i) {
      const auto &c = s.gc[i];
      if (gcBody(c.id) != body)
        continue;
      V3<R> g = -((V3<R>{1, 0, 0} * c.lambda[0] + V3<R>{0, 1, 0} * c.lambda[1]) +
                  V3<R>{0, 0, 1} * c.lambda[2]);
      force.x += g.x;
      force.y += g.y;
      force.z += g.z;
    }
    put(sv.footForces, k, force);
    const V3<R> r = rotate(v.Q(body), V3<R>{sv.sites[f][0], sv.sites[f][1], sv.sites[f][2]});
    const V3<R> vb{s.v[0][body], s.v[1][body], s.v[2][body]};
    put(sv.sitePositions, k, v.X(body) + r);
    put(sv.siteVelocities, k, vb + cross(v.W(body), r));
    const bool contact = norm(force) > R(1e-5);
    if (sv.airTime)
      sv.airTime[k] = contact ? R(0) : sv.airTime[k] + h;
    if (sv.contactTime)
      sv.contactTime[k] = contact ? sv.contactTime[k] + h : R(0);
  }
}

} // namespace duckhip
