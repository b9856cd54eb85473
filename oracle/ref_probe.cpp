// Host driver around the reference's own shared AVBD core (src/cuda/kernel.cuh,
// src/cuda/convex.cuh, src/cuda/model.hpp), compiled in place from the
// reference tree exactly as src/cuda/cpu_bindings.cpp:1-17 compiles it (empty
// __host__/__device__, one scalar namespace per precision).  It exposes a C ABI
// so the oracle's tests and the golden-vector script can read the internal
// state the pybind11 module does not export: the compacted contact list, the
// per-step colours and the joint multipliers.
//
// Test infrastructure only.  Built into oracle/_ref/ by oracle/Makefile when
// the reference tree is present; nothing in the product links it.
// All array arguments are float64 regardless of the probe's precision.
#include "model.hpp"
#include <cstring>
#include <memory>
#include <string>
#define __host__
#define __device__
#define DUCK_NAMESPACE cpu32
#define DUCK_SCALAR float
#include "kernel.cuh"
#undef DUCK_NAMESPACE
#undef DUCK_SCALAR
#define DUCK_NAMESPACE cpu64
#define DUCK_SCALAR double
#include "kernel.cuh"
#undef DUCK_NAMESPACE
#undef DUCK_SCALAR
#undef __host__
#undef __device__

namespace {
thread_local std::string lastError;

struct Base {
  virtual ~Base() = default;
  int bodies = 0, joints = 0;
  bool fp64 = false;
};

template <class S> struct Probe final : Base {
  using Real = typename S::Scalar;
  typename S::ModelType model{};
  std::vector<typename S::Point> points;
  std::unique_ptr<S> state{new S()};
};

using P32 = Probe<cpu32::State>;
using P64 = Probe<cpu64::State>;

template <class S> Probe<S> *make(const char *path, double dt, int iterations) {
  duck::Solver original;
  original.load(path);
  auto *p = new Probe<S>();
  duck_native::convert<S>(original, p->model, p->points, dt, iterations);
  p->state->initialize(&p->model, p->points.data());
  p->bodies = p->model.bodies.size();
  p->joints = p->model.joints.size();
  p->fp64 = std::is_same_v<typename S::Scalar, double>;
  return p;
}

template <class F> int guarded(F &&f) {
  try {
    f();
    return 0;
  } catch (const std::exception &e) {
    lastError = e.what();
    return 1;
  }
}

// Run `f` on the probe with its concrete precision.
template <class F> int visit(void *h, F &&f) {
  auto *base = static_cast<Base *>(h);
  return guarded([&] {
    if (base->fp64)
      f(*static_cast<P64 *>(base));
    else
      f(*static_cast<P32 *>(base));
  });
}

template <class P> using RealOf = typename P::Real;
} // namespace

extern "C" {
const char *probe_last_error() { return lastError.c_str(); }

void *probe_create(const char *path, double dt, int iterations, int fp64) {
  void *out = nullptr;
  guarded([&] {
    if (fp64)
      out = static_cast<Base *>(make<cpu64::State>(path, dt, iterations));
    else
      out = static_cast<Base *>(make<cpu32::State>(path, dt, iterations));
  });
  return out;
}

void probe_destroy(void *h) { delete static_cast<Base *>(h); }

int probe_dims(void *h, int *bodies, int *joints) {
  auto *b = static_cast<Base *>(h);
  *bodies = b->bodies;
  *joints = b->joints;
  return 0;
}

// initialize + resetPose (kernel.cuh:383-420), as resetStates does.
int probe_reset(void *h, const double *q, const double *root) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> qs(p.joints), rs(6);
    for (int i = 0; i < p.joints; ++i)
      qs[i] = R(q[i]);
    for (int i = 0; i < 6; ++i)
      rs[i] = R(root[i]);
    p.state->initialize(&p.model, p.points.data());
    p.state->resetPose(qs.data(), rs.data());
  });
}

// Per-launch parameters of the advance kernel (extension.cu:100-110).
int probe_set_controls(void *h, const double *target, const double *force,
                       double kp, double limit) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    auto &s = *p.state;
    for (int j = 0; j < p.joints; ++j) {
      s.joints[j].target = R(target[j]);
      s.joints[j].kp = R(kp);
      s.joints[j].maxTorque = R(limit);
      s.joints[j].torque = p.model.joints[j].torque;
      s.joints[j].frictionloss = p.model.joints[j].frictionloss;
      s.joints[j].damping = p.model.joints[j].damping;
    }
    s.bodies[1].force = {R(force[0]), R(force[1]), R(force[2])};
  });
}

int probe_set_motor(void *h, const double *motor, const double *force) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> m(3 * p.joints);
    for (int i = 0; i < 3 * p.joints; ++i)
      m[i] = R(motor[i]);
    R f[3] = {R(force[0]), R(force[1]), R(force[2])};
    p.state->setMotor(m.data(), f);
  });
}

int probe_advance(void *h, int substeps) {
  return visit(h, [&](auto &p) { p.state->advance(substeps); });
}

int probe_detect(void *h) {
  return visit(h, [&](auto &p) { p.state->detectContacts(); });
}

int probe_failed(void *h) {
  int out = 0;
  visit(h, [&](auto &p) { out = p.state->failed; });
  return out;
}

// bodies[B*13], joints[J*2], diag[6] as kernel.cuh:555-575.
int probe_snapshot(void *h, double *bodies, double *joints, double *diag) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> b(13 * p.bodies), j(2 * p.joints), d(6);
    p.state->snapshot(b.data(), j.data(), d.data());
    std::copy(b.begin(), b.end(), bodies);
    std::copy(j.begin(), j.end(), joints);
    std::copy(d.begin(), d.end(), diag);
  });
}

// Overwrite one body's pose and velocity (seeded-state parity cases).
int probe_set_body(void *h, int i, const double *x, const double *q,
                   const double *v, const double *w) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    auto &b = p.state->bodies[i];
    b.x = {R(x[0]), R(x[1]), R(x[2])};
    b.q = {R(q[0]), R(q[1]), R(q[2]), R(q[3])};
    b.v = {R(v[0]), R(v[1]), R(v[2])};
    b.w = {R(w[0]), R(w[1]), R(w[2])};
  });
}

// Contact list: ints[n*6] = body, shape, feature, other, otherShape, stick;
// reals[n*26] = local3 anchor3 localB3 tangent1 3 tangent2 3 normal3 friction
// c0 lambda3 penalty3.
enum { CONTACT_INTS = 6, CONTACT_REALS = 26 };
int probe_contacts(void *h, int capacity, int *count, int *ints, double *reals) {
  return visit(h, [&](auto &p) {
    auto &cs = p.state->contacts;
    *count = cs.size();
    for (int k = 0; k < cs.size() && k < capacity; ++k) {
      auto &c = cs[k];
      int *I = ints + CONTACT_INTS * k;
      double *R = reals + CONTACT_REALS * k;
      I[0] = c.body;
      I[1] = c.shape;
      I[2] = c.feature;
      I[3] = c.other;
      I[4] = c.otherShape;
      I[5] = c.stick;
      const decltype(c.local) *vs[] = {&c.local,    &c.anchor,   &c.localB,
                                       &c.tangent1, &c.tangent2, &c.normal};
      for (int v = 0; v < 6; ++v)
        for (int d = 0; d < 3; ++d)
          R[3 * v + d] = (*vs[v])[d];
      R[18] = c.friction;
      R[19] = c.c0;
      for (int d = 0; d < 3; ++d) {
        R[20 + d] = c.lambda[d];
        R[23 + d] = c.penalty[d];
      }
    }
  });
}

int probe_colors(void *h, int *colors, int *count) {
  return visit(h, [&](auto &p) {
    for (int i = 0; i < p.bodies; ++i)
      colors[i] = p.state->colors[i];
    *count = p.state->colorCount;
  });
}

// Joint multipliers: per joint lambda7 penalty7 c0 7 angle0 velocity0 lambdaF
// penaltyF target kp maxTorque torque frictionloss damping (31 values).
int probe_joint_state(void *h, double *out) {
  return visit(h, [&](auto &p) {
    for (int i = 0; i < p.joints; ++i) {
      auto &j = p.state->joints[i];
      double *o = out + 31 * i;
      for (int k = 0; k < 7; ++k) {
        o[k] = j.lambda[k];
        o[7 + k] = j.penalty[k];
        o[14 + k] = j.c0[k];
      }
      double rest[] = {j.angle0, j.velocity0, j.lambdaF,  j.penaltyF,
                       j.target, j.kp,        j.maxTorque, j.torque,
                       j.frictionloss, j.damping};
      std::copy(rest, rest + 10, o + 21);
    }
  });
}

int probe_contact_forces(void *h, int ground_only, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> o(3 * p.bodies);
    p.state->contactForces(o.data(), ground_only != 0);
    std::copy(o.begin(), o.end(), out);
  });
}

int probe_self_contact_stats(void *h, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    R o[2];
    p.state->selfContactStats(o);
    out[0] = o[0];
    out[1] = o[1];
  });
}

int probe_contact_counts(void *h, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    R o[2];
    p.state->contactCounts(o);
    out[0] = o[0];
    out[1] = o[1];
  });
}

int probe_generalized_loads(void *h, const double *offset, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> o(3 * p.joints);
    p.state->generalizedLoads({R(offset[0]), R(offset[1]), R(offset[2])},
                              o.data());
    std::copy(o.begin(), o.end(), out);
  });
}
}
