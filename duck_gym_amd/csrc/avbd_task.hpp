// Control-step kernels of the tensor VecEnv (python/duck_gym/tensor_env.py):
// action clamping and servo targets, and the observation, reward, failure,
// timeout and episode bookkeeping that the reference assembles from ~40 torch
// ops per control step (tensor_env.py:178-219, 221-391).  One lane per
// environment; the root pose and joint state are read straight from the HBM
// state blob, so no [E,B,13] snapshot is materialised.
#pragma once
#include "../../include/duck_hip.h"
#include "avbd_queries.hpp"

namespace duckhip {

enum TaskMode { kTaskStep = 0, kTaskReset = 1 };

DUCK_HD float mexp(float x) { return expf(x); }
DUCK_HD double mexp(double x) { return exp(x); }
DUCK_HD float tsin(float x) { return sinf(x); }
DUCK_HD double tsin(double x) { return sin(x); }

// Observation widths (tensor_env.py:238-258 and the 48-wide rollout layout).
DUCK_HD int taskObsDim(const DuckTask &t, int nj) {
  if (t.kind == DUCK_TASK_STANDING)
    return 10 + 3 * nj;
  if (t.kind == DUCK_TASK_LOCOMOTION)
    return 16 + 3 * nj + (t.velocity_filter ? 2 : 0);
  return 6 + 3 * nj;
}

// The gait reference of hinge j (tensor_env.py:263-277): the episode's
// phase picks two neighbouring rows of the table of the command's direction
// (the first of the largest of +x, -x, +y, -y) and blends them linearly;
// HOME blends into that over the first second.  The operations and their
// order are torch's, in the batch dtype.
template <class R>
DUCK_HD R gaitReference(const DuckTask &t, long long episode, const R *cmd, int j, int nj) {
  const R *table = static_cast<const R *>(t.gait_table);
  const int count = t.gait_phases;
  const R ep = R(episode);
  const R phase = ep * R(t.control_dt) / R(t.gait_period);
  // torch.remainder of a non-negative phase by 1 is fmod; index < count
  // (the clamp only guards the table)
  const R index = fmod(phase, R(1)) * R(count);
  long long lo = static_cast<long long>(index);
  lo = lo < 0 ? 0 : (lo >= count ? count - 1 : lo);
  const R fraction = index - R(lo);
  const R score[4] = {cmd[0], -cmd[0], cmd[1], -cmd[1]};
  int d = 0;
  for (int k = 1; k < 4; ++k)
    d = score[k] > score[d] ? k : d;
  const R a = table[(size_t(d) * count + lo) * nj + j];
  const R b = table[(size_t(d) * count + (lo + 1) % count) * nj + j];
  const R ref = a * (R(1) - fraction) + b * fraction;
  R blend = ep * R(t.control_dt);
  blend = blend < R(0) ? R(0) : (blend > R(1) ? R(1) : blend);
  const R home = R(t.home[j]);
  return home + (ref - home) * blend;
}

// a = clamp(actions, -1, 1); target = clamp(ref + scale a, lower, upper)
// with ref = `reference`, else the gait reference (t.gait), else HOME
// (tensor_env.py:263-283).
template <class R>
__global__ void taskTargetsKernel(DuckTask t, int count, int nj, const R *actions,
                                  const R *reference, const long long *episode, const R *commands,
                                  R *clamped, R *target) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count * nj)
    return;
  int j = i % nj;
  R a = actions[i];
  // torch.clamp propagates NaN; so do these comparisons (NaN fails both).
  a = a < R(-1) ? R(-1) : (a > R(1) ? R(1) : a);
  const int e = i / nj;
  R ref = reference ? reference[i]
                    : (t.gait ? gaitReference<R>(t, episode[e], commands + size_t(e) * 2, j, nj)
                              : R(t.home[j]));
  R v = ref + R(t.action_scale) * a;
  R lo = R(t.lower[j]), hi = R(t.upper[j]);
  v = v < lo ? lo : (v > hi ? hi : v);
  clamped[i] = a;
  target[i] = v;
}

// TensorEnv.reset's inputs from the caller's random draws (tensor_env.py:
// 196-217), each value rounded per operation as the torch expressions are:
// thread i < count * nj writes q[i] = HOME + (u - 0.5) * 0.02 (HOME without
// draws); thread e < count writes the root offset (0, 0, 0.001, (v - 0.5) *
// 0.02, (v' - 0.5) * 0.02, 0) (zeros without draws) and, with a command draw
// (`selected`, or one `direction` for every env), commandsOut = mask ?
// table[direction] * speed : commands.
template <class R>
__global__ void taskResetInputsKernel(DuckTask t, int count, int nj, const unsigned char *mask,
                                      const R *jointDraws, const R *rootDraws,
                                      const long long *selected, int direction, R speed,
                                      const R *commands, R *q, R *roots, R *commandsOut) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count * nj) {
    const R home = R(t.home[i % nj]);
    q[i] = jointDraws ? home + (jointDraws[i] - R(0.5)) * R(0.02) : home;
  }
  if (i >= count)
    return;
  R *r = roots + size_t(i) * 6;
  r[0] = r[1] = r[5] = R(0);
  r[2] = rootDraws ? R(0.001) : R(0);
  r[3] = rootDraws ? (rootDraws[size_t(i) * 2] - R(0.5)) * R(0.02) : R(0);
  r[4] = rootDraws ? (rootDraws[size_t(i) * 2 + 1] - R(0.5)) * R(0.02) : R(0);
  if (selected || direction >= 0) {
    // the direction table [[1, 0], [-1, 0], [0, 1], [0, -1]]
    const int d = selected ? int(selected[i]) : direction;
    const R dx = d == 0 ? R(1) : (d == 1 ? R(-1) : R(0));
    const R dy = d == 2 ? R(1) : (d == 3 ? R(-1) : R(0));
    const bool on = mask[i] != 0;
    commandsOut[size_t(i) * 2] = on ? dx * speed : commands[size_t(i) * 2];
    commandsOut[size_t(i) * 2 + 1] = on ? dy * speed : commands[size_t(i) * 2 + 1];
  }
}

struct TaskBuffers {
  const unsigned char *mask; // reset mode: envs whose bookkeeping restarts
  void *action;              // [E,J] R: this step's clamped action (step) / current actions
  void *lastAction;          // [E,J] R: previous action; step mode overwrites it with action
  const void *commands;      // [E,2] R (locomotion, rollout)
  long long *episode;        // [E]
  void *filtered;            // [E,2] R (locomotion velocity filter)
  float *returns;            // [E]
  void *forces;              // [E,3] R (reset mode zeroes masked rows), may be null
  float *obs;                // [E,D]
  float *reward;             // [E]
  unsigned char *failed, *timeout, *done; // [E]
  void *diag;                // [E,6] R, may be null
};

// What the task kernel reads of a blob, staged in LDS: the 16-byte chunks
// covering the diagnostics through the angular velocities (the targets, force
// and the body poses and velocities lie between them).  A workgroup of 64
// lanes copies its environments' ranges with whole-wave loads (each
// environment's chunks are consecutive, so a load instruction covers a few
// cache lines instead of one line per lane), then each lane computes one
// environment from LDS.
template <class S> constexpr size_t taskStageBegin() { return diagBegin<S>() / 16 * 16; }
template <class S> constexpr size_t taskStageEnd() { return (offsetof(S, w) + sizeof(S::w) + 15) / 16 * 16; }
template <class S> constexpr int taskStageChunks() { return int((taskStageEnd<S>() - taskStageBegin<S>()) / 16); }
// environments per workgroup: as many as 60 KiB of LDS holds, at most 64; the
// record stride in words is the chunks' plus one (odd: the lanes' records
// fall on distinct LDS banks) for a float batch, plus two for a double one
// (whole 8-byte words)
template <class S> constexpr int taskStageStride() {
  return 4 * taskStageChunks<S>() + (sizeof(S::diag[0]) == 4 ? 1 : 2);
}
template <class S> constexpr int taskEnvsPerBlock() {
  return 61440 / (4 * taskStageStride<S>()) > 64 ? 64 : 61440 / (4 * taskStageStride<S>());
}

// The staged fields of one environment (the same values as the blob's).
template <class R, int B, int J, int CG, int CS> struct TaskStage {
  using State = EnvState<R, B, J, CG, CS>;
  const DeviceModel<R> &M;
  const R *r; // the environment's staged words, from taskStageBegin
  static constexpr int at(size_t offset) { return int((offset - taskStageBegin<State>()) / sizeof(R)); }
  DUCK_HD R x(int k, int b) const { return r[at(offsetof(State, x)) + k * B + b]; }
  DUCK_HD R q(int k, int b) const { return r[at(offsetof(State, q)) + k * B + b]; }
  DUCK_HD R v(int k, int b) const { return r[at(offsetof(State, v)) + k * B + b]; }
  DUCK_HD R w(int k, int b) const { return r[at(offsetof(State, w)) + k * B + b]; }
  DUCK_HD R diag(int k) const { return r[at(offsetof(State, diag)) + k]; }
  DUCK_HD Q4<R> Q(int b) const { return {q(0, b), q(1, b), q(2, b), q(3, b)}; }
  DUCK_HD V3<R> W(int b) const { return {w(0, b), w(1, b), w(2, b)}; }
  DUCK_HD V3<R> mv(const R (&a)[3][kMaxModelJoints], int j) const { return {a[0][j], a[1][j], a[2][j]}; }
  DUCK_HD R angle(int j) const {
    return hingeAngle(Q(M.ja[j]), Q(M.jb[j]), mv(M.axisA, j), mv(M.tangentA, j), mv(M.tangentB, j));
  }
};

template <class R, int B, int J, int CG, int CS>
__global__ __launch_bounds__(64) void taskKernel(DuckTask t, int mode, const DeviceModel<R> *model,
                                                 unsigned char *states, long long blobBytes, int count,
                                                 TaskBuffers io) {
  using State = EnvState<R, B, J, CG, CS>;
  constexpr int CH = taskStageChunks<State>(), STRIDE = taskStageStride<State>(),
                TE = taskEnvsPerBlock<State>();
  static_assert(TE >= 1 && (4 * STRIDE) % sizeof(R) == 0 && taskStageBegin<State>() % sizeof(R) == 0,
                "a staged record holds whole words of the batch dtype");
  __shared__ unsigned stage[TE * STRIDE];
  const int e0 = blockIdx.x * TE;
  const int n = count - e0 < TE ? count - e0 : TE;
  // chunk c of environment i is item i CH + c; the lanes take the items in
  // turn, so that a lane's loads are independent and in flight together
#pragma unroll 8
  for (int item = threadIdx.x; item < n * CH; item += 64) {
    const int i = item / CH, c = item - i * CH;
    const uint4 v = reinterpret_cast<const uint4 *>(states + blobBytes * (e0 + i) + taskStageBegin<State>())[c];
    unsigned *dst = stage + i * STRIDE + 4 * c;
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
  }
  __syncthreads();
  const int e = e0 + int(threadIdx.x);
  if (threadIdx.x >= TE || e >= count)
    return;
  const DeviceModel<R> &M = *model;
  const State &s = blobAt<State>(states, blobBytes, e);
  const TaskStage<R, B, J, CG, CS> view{M, reinterpret_cast<const R *>(stage + threadIdx.x * STRIDE)};
  const int nj = M.nj;
  R *act = static_cast<R *>(io.action) + size_t(e) * nj;
  R *last = static_cast<R *>(io.lastAction) + size_t(e) * nj;
  R *filt = io.filtered ? static_cast<R *>(io.filtered) + size_t(e) * 2 : nullptr;
  const R *cmd = io.commands ? static_cast<const R *>(io.commands) + size_t(e) * 2 : nullptr;

  if (mode == kTaskReset && io.mask && io.mask[e]) {
    // tensor_env.py:199-203: restart the episode bookkeeping of reset envs.
    for (int j = 0; j < nj; ++j)
      act[j] = R(0);
    if (filt)
      filt[0] = filt[1] = R(0);
    if (io.forces)
      for (int k = 0; k < 3; ++k)
        static_cast<R *>(io.forces)[size_t(e) * 3 + k] = R(0);
    io.episode[e] = 0;
    io.returns[e] = 0.f;
  }

  // Root frame q = q_body1 (x) conj(root_iquat) (tensor_env.py:140-142, 222).
  const int root = 1;
  Q4<R> qb = view.Q(root);
  Q4<R> iq{R(t.iquat[0]), -R(t.iquat[1]), -R(t.iquat[2]), -R(t.iquat[3])};
  Q4<R> q = qb * iq;
  V3<R> g = rotateInv(q, V3<R>{R(0), R(0), R(-1)});
  V3<R> vel{view.v(0, root), view.v(1, root), view.v(2, root)};
  V3<R> v = rotateInv(q, vel);
  V3<R> w = rotateInv(q, view.W(root));
  R yawC = R(1) - R(2) * (q.y * q.y + q.z * q.z);
  R yawS = R(2) * (q.w * q.z + q.x * q.y);
  R height = view.x(2, root) - R(t.root_height);

  R reward = 0;
  bool failed = false, timeout = false;
  if (mode == kTaskStep) {
    // Failure (tensor_env.py:294-301; the rollout task fails on a fall).
    bool finite = true;
    for (int b = 0; b < M.nb; ++b) {
      for (int k = 0; k < 3; ++k)
        finite = finite && mfinite(view.x(k, b)) && mfinite(view.v(k, b)) && mfinite(view.w(k, b));
      for (int k = 0; k < 4; ++k)
        finite = finite && mfinite(view.q(k, b));
    }
    const R cosHalf = R(cosf(0.5f)); // torch.cos of a float32 0.5
    if (t.kind == DUCK_TASK_ROLLOUT)
      failed = view.x(2, root) < R(t.fall_height);
    else
      failed = g.z > -cosHalf || mabs(height) > R(0.04) || view.diag(kJointError) > R(0.005) ||
               view.diag(kPenetration) > R(0.005);
    failed = failed || s.failed > 0 || !finite;

    R pose = 0, act2 = 0, dact2 = 0;
    for (int j = 0; j < nj; ++j) {
      R d = view.angle(j) - R(t.home[j]);
      pose += d * d;
      act2 += act[j] * act[j];
      R da = act[j] - last[j];
      dact2 += da * da;
    }
    R tilt = g.x * g.x + g.y * g.y;
    R w2 = dot(w, w);
    if (t.kind == DUCK_TASK_STANDING) {
      // tensor_env.py:302-310
      reward = R(1.5) * mexp(R(-20) * tilt) + mexp(R(-2000) * height * height) +
               R(0.5) * mexp(R(-10) * dot(v, v)) - R(0.02) * w2 - R(0.05) * pose -
               R(0.01) * act2 - R(0.02) * dact2;
    } else {
      // tensor_env.py:311-327: world-frame COM velocity against the command.
      R vx = vel.x, vy = vel.y;
      if (t.kind == DUCK_TASK_LOCOMOTION && t.velocity_filter) {
        R alpha = R(t.velocity_alpha);
        filt[0] = (R(1) - alpha) * filt[0] + alpha * vx;
        filt[1] = (R(1) - alpha) * filt[1] + alpha * vy;
        vx = filt[0];
        vy = filt[1];
      }
      R ex = vx - cmd[0], ey = vy - cmd[1];
      R error = ex * ex + ey * ey;
      R sigma = R(t.tracking_sigma);
      reward = R(1) * mexp(R(-20) * tilt) + mexp(R(-2000) * height * height) +
               R(t.tracking_weight) * mexp(-error / (sigma * sigma)) - R(0.1) * w2 -
               R(t.heading_weight) * (R(1) - yawC) - R(0.02) * act2 - R(0.03) * dact2;
    }
    // Gait shaping (tensor_env.py:328-354), at the counter after this step.
    const long long next = io.episode[e] + 1;
    if (t.foot_clearance) {
      // the feet's lowest collision points against a lift that peaks
      // mid-swing; the phase is float32 (an int64 counter times a float)
      const R *pts = static_cast<const R *>(t.foot_point);
      R penalty = 0;
      for (int f = 0; f < 2; ++f) {
        const int fb = t.feet[f];
        const V3<R> p{view.x(0, fb), view.x(1, fb), view.x(2, fb)};
        const Q4<R> qf = view.Q(fb);
        // inverse_rotate(q, up) (tensor_env.py:21-23)
        const V3<R> up{R(0), R(0), R(1)}, u{-qf.x, -qf.y, -qf.z};
        const V3<R> tt = cross(u, up) * R(2);
        const V3<R> localUp = (up + tt * qf.w) + cross(u, tt);
        R lowest = R(0);
        for (int k = 0; k < t.foot_points; ++k) {
          const R *v = pts + (size_t(f) * t.foot_points + k) * 3;
          const R h = (v[0] * localUp.x + v[1] * localUp.y + v[2] * localUp.z) + p.z;
          lowest = k == 0 || h < lowest ? h : lowest;
        }
        float phase = float(next) * float(t.control_dt) / float(t.gait_period) + (f ? 0.5f : 0.0f);
        phase = fmodf(phase, 1.0f);
        float swing = (phase - 0.6f) / 0.4f;
        swing = swing < 0.0f ? 0.0f : (swing > 1.0f ? 1.0f : swing);
        const float sw = sinf(float(3.14159265358979323846) * swing);
        const R desired = R(float(t.gait_lift) * (sw * sw));
        const R gap = (lowest < R(0) ? R(0) : lowest) - desired;
        penalty += gap * gap;
      }
      reward -= R(20000) * penalty;
    }
    if (t.load_transfer) {
      // vertical contact force of each foot, in body weights, against a
      // sinusoidal left/right split
      const R cycle = (R(io.episode[e]) + R(1)) * R(t.control_dt) / R(t.gait_period);
      const R left = R(0.5) + R(0.5) * tsin(R(2 * 3.14159265358979323846) * (cycle - R(0.05)));
      R penalty = 0;
      for (int f = 0; f < 2; ++f) {
        R force = contactForceZ(s, t.feet[f]) / R(t.weight);
        force = force < R(0) ? R(0) : (force > R(3) ? R(3) : force);
        const R d = force - (f ? R(1) - left : left);
        penalty += d * d;
      }
      reward -= R(3) * penalty;
    }
    reward = (failed ? R(-2) : reward) * R(t.control_dt);
    long long ep = next;
    io.episode[e] = ep;
    io.returns[e] += float(reward);
    timeout = ep >= t.max_episode_length && !failed;
    io.reward[e] = float(reward);
    io.failed[e] = failed;
    io.timeout[e] = timeout;
    io.done[e] = failed || timeout;
    for (int j = 0; j < nj; ++j)
      last[j] = act[j];
    if (io.diag) {
      R *d = static_cast<R *>(io.diag) + size_t(e) * 6;
      d[0] = view.diag(kJointError);
      d[1] = view.diag(kPenetration);
      d[2] = view.diag(kContacts);
      d[3] = view.diag(kConverged);
      d[4] = view.diag(kAxisError);
      d[5] = R(s.failed);
    }
  }

  // Observation (tensor_env.py:238-258), cast to float32.
  float *o = io.obs + size_t(e) * taskObsDim(t, nj);
  int k = 0;
  o[k++] = float(g.x);
  o[k++] = float(g.y);
  o[k++] = float(g.z);
  if (t.kind != DUCK_TASK_ROLLOUT) {
    o[k++] = float(v.x);
    o[k++] = float(v.y);
    o[k++] = float(v.z);
  }
  o[k++] = float(w.x);
  o[k++] = float(w.y);
  o[k++] = float(w.z);
  if (t.kind != DUCK_TASK_ROLLOUT)
    o[k++] = float(height);
  for (int j = 0; j < nj; ++j)
    o[k + j] = float(view.angle(j) - R(t.home[j]));
  k += nj;
  for (int j = 0; j < nj; ++j) {
    R rate = dot(view.W(M.jb[j]) - view.W(M.ja[j]), rotate(view.Q(M.ja[j]), view.mv(M.axisA, j)));
    o[k + j] = float(R(0.1) * rate);
  }
  k += nj;
  for (int j = 0; j < nj; ++j)
    o[k + j] = float(act[j]);
  k += nj;
  if (t.kind == DUCK_TASK_LOCOMOTION) {
    // (episode * control_dt) * (2 pi / period), the factor formed in double.
    R phase = R(io.episode[e]) * R(t.control_dt) * R(2 * 3.14159265358979323846 / t.gait_period);
    o[k++] = float(cmd[0]);
    o[k++] = float(cmd[1]);
    o[k++] = float(yawC);
    o[k++] = float(yawS);
    o[k++] = float(msin(phase));
    o[k++] = float(mcos(phase));
    if (t.velocity_filter) {
      o[k++] = float(filt[0]);
      o[k++] = float(filt[1]);
    }
  }
}

} // namespace duckhip
