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

} // namespace duckhip
