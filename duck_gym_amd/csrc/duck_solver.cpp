// duck::Solver (include/duck/solver.hpp) over the C ABI of this library.
// step() and stepAll() hand the public members to duck_sequential_step (the
// explicit-sequential step of src/solver.cpp, one GPU thread per
// environment) and read them back; stepImplicit() writes them into a
// one-environment float64 device batch of the CudaBatch step and reads it
// back.
#include "../../include/duck/solver.hpp"
#include "../../include/duck_hip.h"
#include "duck_model.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cctype>
#include <exception>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <sstream>

namespace duck {
namespace {

// Indices into duck_state_layout's descriptor.
enum LayoutIndex {
  kB, kJ, kCG, kCS, kReal, kBlob, kHeader, kX, kQ, kV, kW, kMass, kInertia, kForce, kLambda,
  kPenalty, kLambdaF, kPenaltyF, kTarget, kKp, kMaxTorque, kTorque, kFrictionloss, kDamping,
  kDiag, kFriction, kFailed, kNgc, kNsc, kColors, kColorCount, kGc, kGcBytes, kSc, kScBytes,
  kGcId, kGcLocal, kGcAnchor, kGcC0, kGcLambda, kGcPenalty, kLayoutSize = 51
};

Vec3 vec(const double v[3]) { return {v[0], v[1], v[2]}; }

// Body-frame candidate points and bounding radius of a shape (solver.cpp:
// 128-148): a box's eight corners, a hull's vertices, none for a sphere or
// a capsule, whose radius is |centre| plus its size(s).
void shapePoints(Shape &s) {
  s.localPoints.clear();
  if (s.type == 1) {
    for (int i = 0; i < 8; ++i)
      s.localPoints.push_back(s.center + rotate(s.q, Vec3{(i & 1 ? 1 : -1) * s.size.x,
                                                         (i & 2 ? 1 : -1) * s.size.y,
                                                         (i & 4 ? 1 : -1) * s.size.z}));
  } else if (s.type == 3) {
    for (auto v : s.vertices)
      s.localPoints.push_back(s.center + rotate(s.q, v));
  }
  s.boundingRadius = 0;
  for (auto p : s.localPoints)
    s.boundingRadius = std::max(s.boundingRadius, norm(p));
  if (s.type == 0)
    s.boundingRadius = norm(s.center) + s.size.x;
  if (s.type == 2)
    s.boundingRadius = norm(s.center) + s.size.x + s.size.y;
}

void fail(int code) {
  const std::string message = duck_last_error();
  if (code == DUCK_ERR_MODEL)
    throw std::invalid_argument(message);
  throw std::runtime_error(message);
}
void hip(hipError_t err, const char *what) {
  if (err != hipSuccess)
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

} // namespace

struct Solver::Device {
  void *handle = nullptr;
  void *staging = nullptr; // one state blob in device memory
  std::string signature;
  long long layout[kLayoutSize] = {};
  std::vector<unsigned char> blob;
  ~Device() {
    if (handle)
      duck_destroy(handle);
    if (staging)
      (void)hipFree(staging);
  }
  template <class T> T *at(long long offset) { return reinterpret_cast<T *>(blob.data() + offset); }
  double *real(int field, int component, int stride) {
    return at<double>(layout[field]) + size_t(component) * stride;
  }
};

Solver::Solver() = default;
Solver::~Solver() = default;
Solver::Solver(const Solver &o)
    : options(o.options), bodies(o.bodies), joints(o.joints), shapes(o.shapes),
      collisionPairs(o.collisionPairs), contacts(o.contacts), diagnostics(o.diagnostics),
      initialBodies(o.initialBodies), initialJoints(o.initialJoints),
      bodyContacts(o.bodyContacts) {}
Solver &Solver::operator=(const Solver &o) {
  if (this != &o) {
    options = o.options;
    bodies = o.bodies;
    joints = o.joints;
    shapes = o.shapes;
    collisionPairs = o.collisionPairs;
    contacts = o.contacts;
    diagnostics = o.diagnostics;
    initialBodies = o.initialBodies;
    initialJoints = o.initialJoints;
    bodyContacts = o.bodyContacts;
    device.reset();
  }
  return *this;
}

void Solver::load(const std::string &path) {
  duckhip::HostModel m = duckhip::parseModel(path);
  options.gravity = vec(m.gravity);
  options.ground = m.ground != 0;
  bodies.assign(m.bodies.size(), Body{});
  for (size_t i = 0; i < bodies.size(); ++i) {
    const auto &h = m.bodies[i];
    Body &b = bodies[i];
    b.name = h.name;
    b.mass = h.mass;
    b.inertia = vec(h.inertia);
    b.x = vec(h.x);
    b.q = {h.q[0], h.q[1], h.q[2], h.q[3]};
    b.v = vec(h.v);
    b.w = vec(h.w);
  }
  joints.assign(m.joints.size(), Joint{});
  for (size_t i = 0; i < joints.size(); ++i) {
    const auto &h = m.joints[i];
    Joint &j = joints[i];
    j.name = h.name;
    j.a = h.a;
    j.b = h.b;
    j.ra = vec(h.ra);
    j.rb = vec(h.rb);
    j.axisA = vec(h.axisA);
    j.axisB = vec(h.axisB);
    j.tangentA = vec(h.tangentA);
    j.tangentB = vec(h.tangentB);
    j.limited = h.limited != 0;
    j.lo = h.lo;
    j.hi = h.hi;
    j.damping = h.damping;
    j.armature = h.armature;
    j.frictionloss = h.frictionloss;
    j.torque = h.torque;
    j.kp = h.kp;
    j.target = h.target;
    j.maxTorque = h.maxTorque;
    // penalty floors: 1000 on anchor rows, 1 on angular rows (model.hpp)
    for (int k = 0; k < 7; ++k)
      j.penalty[k] = k < 3 ? 1000 : 1;
  }
  shapes.assign(m.shapes.size(), Shape{});
  for (size_t i = 0; i < shapes.size(); ++i) {
    const auto &h = m.shapes[i];
    Shape &s = shapes[i];
    s.body = h.body;
    s.type = h.type;
    s.center = vec(h.center);
    s.q = {h.q[0], h.q[1], h.q[2], h.q[3]};
    s.size = vec(h.size);
    s.friction = h.friction;
    s.ground = h.ground != 0;
    for (size_t v = 0; v + 2 < h.vertices.size(); v += 3)
      s.vertices.push_back({h.vertices[v], h.vertices[v + 1], h.vertices[v + 2]});
    shapePoints(s);
  }
  collisionPairs.assign(m.pairs.size(), CollisionPair{});
  for (size_t i = 0; i < m.pairs.size(); ++i)
    collisionPairs[i] = {m.pairs[i].a, m.pairs[i].b, m.pairs[i].friction};
  contacts.clear();
  bodyContacts.clear();
  diagnostics = {};
  initialBodies = bodies;
  initialJoints = joints;
  device.reset();
}

void Solver::reset() {
  bodies = initialBodies;
  joints = initialJoints;
  contacts.clear();
  bodyContacts.clear();
  diagnostics = {};
}

double Solver::angle(const Joint &j) const {
  const Body &a = bodies.at(j.a), &b = bodies.at(j.b);
  const Vec3 axis = rotate(a.q, j.axisA), ta = rotate(a.q, j.tangentA),
             tb = rotate(b.q, j.tangentB);
  // signed angle from ta to tb about the axis
  return std::atan2(dot(axis, cross(ta, tb)), dot(ta, tb));
}

void Solver::evaluateJoint(const Joint &j, std::array<double, 7> &C, std::array<V6, 7> &JA,
                           std::array<V6, 7> &JB) const {
  const Body &a = bodies.at(j.a), &b = bodies.at(j.b);
  const Vec3 ra = rotate(a.q, j.ra), rb = rotate(b.q, j.rb);
  const Vec3 gap = a.x + ra - b.x - rb; // left to right, as solver.cpp:192
  // anchors coincide: one row per world axis e, C = gap . e, with
  // d(gap)/d(x_a, theta_a) = (e, ra x e) and the opposite on b
  for (int k = 0; k < 3; ++k) {
    Vec3 e{};
    e[k] = 1;
    C[k] = gap[k];
    JA[k] = row(e, cross(ra, e));
    JB[k] = row(-e, cross(e, rb));
  }
  // axes align: b's axis has no component along a's two tangents
  const Vec3 axis = rotate(a.q, j.axisA), axisB = rotate(b.q, j.axisB);
  const Vec3 t[2] = {rotate(a.q, j.tangentA), cross(axis, rotate(a.q, j.tangentA))};
  for (int k = 0; k < 2; ++k) {
    C[3 + k] = dot(t[k], axisB);
    JA[3 + k] = row({}, cross(t[k], axisB));
    JB[3 + k] = row({}, cross(axisB, t[k]));
  }
  // limits: angle - lo >= 0 and hi - angle >= 0
  const double q = angle(j);
  C[5] = q - j.lo;
  C[6] = j.hi - q;
  JA[5] = row({}, -axis);
  JB[5] = row({}, axis);
  JA[6] = row({}, axis);
  JB[6] = row({}, -axis);
}

namespace {

std::ostream &put(std::ostream &o, Vec3 v) { return o << ' ' << v.x << ' ' << v.y << ' ' << v.z; }
std::ostream &put(std::ostream &o, Quat q) {
  return o << ' ' << q.w << ' ' << q.x << ' ' << q.y << ' ' << q.z;
}

// The model as `.duck` v2 text.  With `state`, body poses and velocities and
// the hinges' control fields are written; without, they are left out (the
// signature of what the device batch's model depends on).
std::string modelText(const Solver &s, bool state) {
  std::ostringstream o;
  o << std::setprecision(17);
  o << "DUCK_MODEL 2 " << s.bodies.size() << ' ' << s.joints.size() << ' ' << s.shapes.size()
    << '\n';
  put(o, s.options.gravity) << ' ' << (s.options.ground ? 1 : 0) << '\n';
  for (const Body &b : s.bodies) {
    o << b.name << ' ' << b.mass;
    put(o, b.inertia);
    if (state) {
      put(o, b.x);
      put(o, b.q);
      put(o, b.v);
      put(o, b.w);
    }
    o << '\n';
  }
  for (const Joint &j : s.joints) {
    o << j.name << ' ' << j.a << ' ' << j.b;
    put(o, j.ra);
    put(o, j.rb);
    put(o, j.axisA);
    put(o, j.axisB);
    put(o, j.tangentA);
    put(o, j.tangentB);
    o << ' ' << (j.limited ? 1 : 0) << ' ' << j.lo << ' ' << j.hi;
    if (state)
      o << ' ' << j.damping << ' ' << j.armature << ' ' << j.frictionloss << ' ' << j.torque
        << ' ' << j.kp << ' ' << j.target << ' ' << j.maxTorque;
    else
      o << ' ' << j.armature;
    o << '\n';
  }
  for (const Shape &sh : s.shapes) {
    o << sh.body << ' ' << sh.type;
    put(o, sh.center);
    put(o, sh.q);
    put(o, sh.size);
    o << ' ' << sh.friction << ' ' << sh.vertices.size();
    for (auto v : sh.vertices)
      put(o, v);
    o << ' ' << (sh.ground ? 1 : 0) << '\n';
  }
  o << s.collisionPairs.size() << '\n';
  for (const auto &p : s.collisionPairs)
    o << p.a << ' ' << p.b << ' ' << p.friction << '\n';
  return o.str();
}

} // namespace

namespace {

// One Solver's structs for duck_sequential_step.
struct SequentialStage {
  std::vector<DuckSeqBody> bodies;
  std::vector<DuckSeqJoint> joints;
  std::vector<DuckSeqShape> shapes;
  std::vector<double> points;
  std::vector<DuckSeqContact> contacts;
  DuckSeqEnv env{};
};

void put3(double *d, Vec3 v) {
  d[0] = v.x;
  d[1] = v.y;
  d[2] = v.z;
}
void put4(double *d, Quat q) {
  d[0] = q.w;
  d[1] = q.x;
  d[2] = q.y;
  d[3] = q.z;
}
Vec3 get3(const double *d) { return {d[0], d[1], d[2]}; }
Quat get4(const double *d) { return {d[0], d[1], d[2], d[3]}; }

void stage(const Solver &s, SequentialStage &st) {
  const Options &o = s.options;
  DuckSeqOptions &so = st.env.options;
  so.dt = o.dt;
  so.alpha = o.alpha;
  so.gamma = o.gamma;
  so.beta_linear = o.betaLinear;
  so.beta_angular = o.betaAngular;
  so.tolerance = o.tolerance;
  put3(so.gravity, o.gravity);
  so.iterations = o.iterations;
  so.ground = o.ground ? 1 : 0;
  st.bodies.assign(s.bodies.size(), DuckSeqBody{});
  for (size_t i = 0; i < s.bodies.size(); ++i) {
    const Body &b = s.bodies[i];
    DuckSeqBody &d = st.bodies[i];
    d.mass = b.mass;
    put3(d.inertia, b.inertia);
    put3(d.x, b.x);
    put3(d.v, b.v);
    put3(d.w, b.w);
    put3(d.x0, b.x0);
    put3(d.xp, b.xp);
    put3(d.force, b.force);
    put4(d.q, b.q);
    put4(d.q0, b.q0);
    put4(d.qp, b.qp);
  }
  st.joints.assign(s.joints.size(), DuckSeqJoint{});
  for (size_t i = 0; i < s.joints.size(); ++i) {
    const Joint &j = s.joints[i];
    DuckSeqJoint &d = st.joints[i];
    d.a = j.a;
    d.b = j.b;
    d.limited = j.limited ? 1 : 0;
    put3(d.ra, j.ra);
    put3(d.rb, j.rb);
    put3(d.axis_a, j.axisA);
    put3(d.axis_b, j.axisB);
    put3(d.tangent_a, j.tangentA);
    put3(d.tangent_b, j.tangentB);
    d.lo = j.lo;
    d.hi = j.hi;
    d.damping = j.damping;
    d.armature = j.armature;
    d.frictionloss = j.frictionloss;
    d.lambda_f = j.lambdaF;
    d.penalty_f = j.penaltyF;
    d.torque = j.torque;
    d.kp = j.kp;
    d.target = j.target;
    d.max_torque = j.maxTorque;
    d.angle0 = j.angle0;
    d.velocity0 = j.velocity0;
    for (int k = 0; k < 7; ++k) {
      d.lambda[k] = j.lambda[k];
      d.penalty[k] = j.penalty[k];
      d.c0[k] = j.c0[k];
    }
  }
  st.shapes.assign(s.shapes.size(), DuckSeqShape{});
  st.points.clear();
  for (size_t i = 0; i < s.shapes.size(); ++i) {
    const Shape &sh = s.shapes[i];
    DuckSeqShape &d = st.shapes[i];
    d.body = sh.body;
    d.type = sh.type;
    d.ground = sh.ground ? 1 : 0;
    d.first_point = int(st.points.size() / 3);
    d.num_points = int(sh.localPoints.size());
    for (Vec3 p : sh.localPoints) {
      st.points.push_back(p.x);
      st.points.push_back(p.y);
      st.points.push_back(p.z);
    }
    put3(d.center, sh.center);
    put3(d.size, sh.size);
    put4(d.q, sh.q);
    d.friction = sh.friction;
    d.bounding_radius = sh.boundingRadius;
  }
  const size_t capacity = std::max(s.contacts.size(), 4 * s.shapes.size());
  st.contacts.assign(capacity, DuckSeqContact{});
  for (size_t i = 0; i < s.contacts.size(); ++i) {
    const Contact &c = s.contacts[i];
    DuckSeqContact &d = st.contacts[i];
    d.body = c.body;
    d.shape = c.shape;
    d.feature = c.feature;
    d.stick = c.stick ? 1 : 0;
    put3(d.local, c.local);
    put3(d.anchor, c.anchor);
    d.radius = c.radius;
    d.friction = c.friction;
    d.c0 = c.c0;
    for (int k = 0; k < 3; ++k) {
      d.lambda[k] = c.lambda[k];
      d.penalty[k] = c.penalty[k];
    }
  }
  DuckSeqEnv &e = st.env;
  e.num_bodies = int(st.bodies.size());
  e.num_joints = int(st.joints.size());
  e.num_shapes = int(st.shapes.size());
  e.num_points = int(st.points.size() / 3);
  e.num_contacts = int(s.contacts.size());
  e.contact_capacity = int(capacity);
  e.bodies = st.bodies.data();
  e.joints = st.joints.data();
  e.shapes = st.shapes.data();
  e.points = st.points.data();
  e.contacts = st.contacts.data();
}

void unstage(const SequentialStage &st, Solver &s) {
  for (size_t i = 0; i < s.bodies.size(); ++i) {
    Body &b = s.bodies[i];
    const DuckSeqBody &d = st.bodies[i];
    b.x = get3(d.x);
    b.v = get3(d.v);
    b.w = get3(d.w);
    b.x0 = get3(d.x0);
    b.xp = get3(d.xp);
    b.q = get4(d.q);
    b.q0 = get4(d.q0);
    b.qp = get4(d.qp);
  }
  for (size_t i = 0; i < s.joints.size(); ++i) {
    Joint &j = s.joints[i];
    const DuckSeqJoint &d = st.joints[i];
    j.lambdaF = d.lambda_f;
    j.penaltyF = d.penalty_f;
    j.angle0 = d.angle0;
    j.velocity0 = d.velocity0;
    for (int k = 0; k < 7; ++k) {
      j.lambda[k] = d.lambda[k];
      j.penalty[k] = d.penalty[k];
      j.c0[k] = d.c0[k];
    }
  }
  s.contacts.assign(st.env.num_contacts, Contact{});
  for (int i = 0; i < st.env.num_contacts; ++i) {
    const DuckSeqContact &d = st.contacts[i];
    Contact &c = s.contacts[i];
    c.body = d.body;
    c.shape = d.shape;
    c.feature = d.feature;
    c.stick = d.stick != 0;
    c.local = get3(d.local);
    c.anchor = get3(d.anchor);
    c.radius = d.radius;
    c.friction = d.friction;
    c.c0 = d.c0;
    for (int k = 0; k < 3; ++k) {
      c.lambda[k] = d.lambda[k];
      c.penalty[k] = d.penalty[k];
    }
  }
  const DuckSeqDiagnostics &g = st.env.diagnostics;
  s.diagnostics.jointError = g.joint_error;
  s.diagnostics.axisError = g.axis_error;
  s.diagnostics.penetration = g.penetration;
  s.diagnostics.update = g.update;
  s.diagnostics.contacts = g.contacts;
  s.diagnostics.iterations = g.iterations;
  s.diagnostics.converged = g.converged != 0;
}

// What the reference's step throws before it changes anything
// (solver.cpp:316-320).
void checkSequential(const Solver &s) {
  if (!s.collisionPairs.empty())
    throw std::runtime_error("Body contacts require the shared CpuBatch/CUDA solver");
  const Options &o = s.options;
  if (!(o.dt > 0) || o.iterations < 1 || o.alpha < 0 || o.alpha >= 1 || o.gamma <= 0 ||
      o.gamma >= 1)
    throw std::runtime_error("Invalid solver options");
}

// The exception the reference's step throws where the device step stopped.
void throwFault(int status) {
  switch (status) {
  case DUCK_SEQ_HESSIAN:
    throw std::runtime_error("Non-positive local Hessian");
  case DUCK_SEQ_NONFINITE:
    throw std::runtime_error("Non-finite state");
  case DUCK_SEQ_QUATERNION:
    throw std::runtime_error("Zero quaternion");
  default:
    throw std::runtime_error("sequential step: unknown fault " + std::to_string(status));
  }
}

// Solver::step of solvers[0..n) in one launch, with the outcome of stepping
// them in order: an environment the reference would reject stops the list
// there, and the first environment that faults is written back and thrown.
void stepSolvers(Solver *const *solvers, int n) {
  int stepped = n;
  std::exception_ptr rejected;
  for (int i = 0; i < n; ++i) {
    try {
      checkSequential(*solvers[i]);
    } catch (...) {
      rejected = std::current_exception();
      stepped = i;
      break;
    }
  }
  if (stepped > 0) {
    std::vector<SequentialStage> stages(stepped);
    std::vector<DuckSeqEnv> envs(stepped);
    for (int i = 0; i < stepped; ++i) {
      stage(*solvers[i], stages[i]);
      envs[i] = stages[i].env;
    }
    int gpu = 0;
    hip(hipGetDevice(&gpu), "hipGetDevice");
    if (duck_sequential_step(envs.data(), stepped, 1, gpu) != DUCK_OK)
      throw std::runtime_error(duck_last_error());
    for (int i = 0; i < stepped; ++i) {
      stages[i].env = envs[i];
      unstage(stages[i], *solvers[i]);
      if (envs[i].status != DUCK_SEQ_OK)
        throwFault(envs[i].status);
    }
  }
  if (rejected)
    std::rethrow_exception(rejected);
}

} // namespace

void Solver::step() {
  Solver *self = this;
  stepSolvers(&self, 1);
}

void stepAll(std::vector<Solver> &environments) {
  std::vector<Solver *> all(environments.size());
  for (size_t i = 0; i < environments.size(); ++i)
    all[i] = &environments[i];
  stepSolvers(all.data(), int(all.size()));
}

void Solver::stepImplicit() {
  const Options defaults;
  if (options.alpha != defaults.alpha || options.gamma != defaults.gamma ||
      options.betaLinear != defaults.betaLinear || options.betaAngular != defaults.betaAngular ||
      options.tolerance != defaults.tolerance)
    throw std::invalid_argument("duck::Solver::step runs alpha 0.9, gamma 0.99, beta 1e7/1e5 "
                                "and tolerance 1e-7 only");
  if (!(options.dt > 0) || options.iterations < 1)
    throw std::invalid_argument("Invalid batch parameters");
  for (size_t i = 0; i < bodies.size(); ++i)
    if (i != 1 && (bodies[i].force.x != 0 || bodies[i].force.y != 0 || bodies[i].force.z != 0))
      throw std::invalid_argument("duck::Solver::step applies a force to the root body only");
  auto token = [](const std::string &name) {
    if (name.empty())
      return false;
    for (char c : name)
      if (std::isspace(static_cast<unsigned char>(c)))
        return false;
    return true;
  };
  for (const Body &b : bodies)
    if (!token(b.name))
      throw std::invalid_argument("body names are single non-empty tokens");
  for (const Joint &j : joints)
    if (!token(j.name))
      throw std::invalid_argument("hinge names are single non-empty tokens");

  std::ostringstream sig;
  sig << std::setprecision(17) << options.dt << ' ' << options.iterations << '\n'
      << modelText(*this, false);
  if (!device || device->signature != sig.str()) {
    device.reset();
    auto d = std::make_unique<Device>();
    int gpu = 0;
    hip(hipGetDevice(&gpu), "hipGetDevice");
    const std::string text = modelText(*this, true);
    const int code =
        duck_create_text(text.c_str(), 1, options.dt, options.iterations, gpu, 64, 0, &d->handle);
    if (code)
      fail(code);
    if (int c = duck_state_layout(d->handle, d->layout))
      fail(c);
    d->blob.assign(size_t(d->layout[kBlob]), 0);
    hip(hipMalloc(&d->staging, d->blob.size()), "hipMalloc(state)");
    if (int c = duck_export_state(d->handle, d->staging, nullptr))
      fail(c);
    hip(hipMemcpy(d->blob.data(), d->staging, d->blob.size(), hipMemcpyDeviceToHost), "download");
    d->signature = sig.str();
    device = std::move(d);
  }
  Device &d = *device;
  const int B = int(d.layout[kB]), J = int(d.layout[kJ]), CG = int(d.layout[kCG]),
            CS = int(d.layout[kCS]);
  const int nb = bodies.size(), nj = joints.size();
  if (int(contacts.size()) > CG)
    throw std::invalid_argument("more ground contacts than the state holds");

  // ---- the public state into the blob ----
  for (int i = 0; i < nb; ++i) {
    const Body &b = bodies[i];
    d.real(kMass, 0, 0)[i] = b.mass;
    for (int k = 0; k < 3; ++k) {
      d.real(kInertia, k, B)[i] = b.inertia[k];
      d.real(kX, k, B)[i] = b.x[k];
      d.real(kV, k, B)[i] = b.v[k];
      d.real(kW, k, B)[i] = b.w[k];
    }
    const double q[4] = {b.q.w, b.q.x, b.q.y, b.q.z};
    for (int k = 0; k < 4; ++k)
      d.real(kQ, k, B)[i] = q[k];
  }
  for (int k = 0; k < 3; ++k)
    d.real(kForce, 0, 0)[k] = nb > 1 ? bodies[1].force[k] : 0;
  for (int i = 0; i < nj; ++i) {
    const Joint &j = joints[i];
    for (int k = 0; k < 7; ++k) {
      d.real(kLambda, k, J)[i] = j.lambda[k];
      d.real(kPenalty, k, J)[i] = j.penalty[k];
    }
    d.real(kLambdaF, 0, 0)[i] = j.lambdaF;
    d.real(kPenaltyF, 0, 0)[i] = j.penaltyF;
    d.real(kTarget, 0, 0)[i] = j.target;
    d.real(kKp, 0, 0)[i] = j.kp;
    d.real(kMaxTorque, 0, 0)[i] = j.maxTorque;
    d.real(kTorque, 0, 0)[i] = j.torque;
    d.real(kFrictionloss, 0, 0)[i] = j.frictionloss;
    d.real(kDamping, 0, 0)[i] = j.damping;
  }
  *d.real(kFriction, 0, 0) = -1; // shape frictions
  *d.at<int>(d.layout[kFailed]) = 0;
  *d.at<int>(d.layout[kNgc]) = int(contacts.size());
  for (size_t c = 0; c < contacts.size(); ++c) {
    const Contact &ct = contacts[c];
    unsigned char *base = d.blob.data() + d.layout[kGc] + c * d.layout[kGcBytes];
    std::memset(base, 0, size_t(d.layout[kGcBytes]));
    const int id = ct.shape | (ct.body << 6) | (ct.feature << 12) |
                   (ct.stick ? int(0x80000000u) : 0);
    std::memcpy(base + d.layout[kGcId], &id, sizeof(id));
    double *local = reinterpret_cast<double *>(base + d.layout[kGcLocal]);
    double *anchor = reinterpret_cast<double *>(base + d.layout[kGcAnchor]);
    double *c0 = reinterpret_cast<double *>(base + d.layout[kGcC0]);
    double *lam = reinterpret_cast<double *>(base + d.layout[kGcLambda]);
    double *pen = reinterpret_cast<double *>(base + d.layout[kGcPenalty]);
    for (int k = 0; k < 3; ++k) {
      local[k] = ct.local[k];
      lam[k] = ct.lambda[k];
      pen[k] = ct.penalty[k];
    }
    anchor[0] = ct.anchor.x;
    anchor[1] = ct.anchor.y;
    *c0 = ct.c0;
  }
  const size_t scBytes = size_t(d.layout[kScBytes]);
  const int nsc = int(bodyContacts.size() / scBytes);
  if (nsc > CS)
    throw std::invalid_argument("more body contacts than the state holds");
  *d.at<int>(d.layout[kNsc]) = nsc;
  if (nsc)
    std::memcpy(d.blob.data() + d.layout[kSc], bodyContacts.data(), bodyContacts.size());

  // ---- one step on the device ----
  hip(hipMemcpy(d.staging, d.blob.data(), d.blob.size(), hipMemcpyHostToDevice), "upload");
  if (int c = duck_import_state(d.handle, d.staging, nullptr))
    fail(c);
  if (int c = duck_advance(d.handle, 1, nullptr))
    fail(c);
  if (int c = duck_export_state(d.handle, d.staging, nullptr))
    fail(c);
  hip(hipMemcpy(d.blob.data(), d.staging, d.blob.size(), hipMemcpyDeviceToHost), "download");
  if (*d.at<int>(d.layout[kFailed]))
    throw std::runtime_error("Non-finite state after the step");

  // ---- and back ----
  for (int i = 0; i < nb; ++i) {
    Body &b = bodies[i];
    b.x0 = b.x;
    b.q0 = b.q;
    for (int k = 0; k < 3; ++k) {
      b.x[k] = d.real(kX, k, B)[i];
      b.v[k] = d.real(kV, k, B)[i];
      b.w[k] = d.real(kW, k, B)[i];
    }
    b.q = {d.real(kQ, 0, B)[i], d.real(kQ, 1, B)[i], d.real(kQ, 2, B)[i], d.real(kQ, 3, B)[i]};
  }
  for (int i = 0; i < nj; ++i) {
    Joint &j = joints[i];
    for (int k = 0; k < 7; ++k) {
      j.lambda[k] = d.real(kLambda, k, J)[i];
      j.penalty[k] = d.real(kPenalty, k, J)[i];
    }
    j.lambdaF = d.real(kLambdaF, 0, 0)[i];
    j.penaltyF = d.real(kPenaltyF, 0, 0)[i];
  }
  const int ngc = *d.at<int>(d.layout[kNgc]);
  contacts.assign(ngc, Contact{});
  for (int c = 0; c < ngc; ++c) {
    const unsigned char *base = d.blob.data() + d.layout[kGc] + c * d.layout[kGcBytes];
    int id;
    std::memcpy(&id, base + d.layout[kGcId], sizeof(id));
    const double *local = reinterpret_cast<const double *>(base + d.layout[kGcLocal]);
    const double *anchor = reinterpret_cast<const double *>(base + d.layout[kGcAnchor]);
    const double *lam = reinterpret_cast<const double *>(base + d.layout[kGcLambda]);
    const double *pen = reinterpret_cast<const double *>(base + d.layout[kGcPenalty]);
    Contact &ct = contacts[c];
    ct.shape = id & 63;
    ct.body = (id >> 6) & 63;
    ct.feature = (id >> 12) & 0x7ffff;
    ct.stick = id < 0;
    ct.local = {local[0], local[1], local[2]};
    ct.anchor = {anchor[0], anchor[1], 0};
    ct.c0 = *reinterpret_cast<const double *>(base + d.layout[kGcC0]);
    for (int k = 0; k < 3; ++k) {
      ct.lambda[k] = lam[k];
      ct.penalty[k] = pen[k];
    }
    ct.friction = shapes.at(ct.shape).friction;
  }
  const int nscOut = *d.at<int>(d.layout[kNsc]);
  bodyContacts.assign(d.blob.data() + d.layout[kSc],
                      d.blob.data() + d.layout[kSc] + size_t(nscOut) * scBytes);
  const double *diag = d.real(kDiag, 0, 0);
  diagnostics.jointError = diag[0];
  diagnostics.penetration = diag[1];
  diagnostics.contacts = int(diag[2]);
  diagnostics.converged = diag[3] != 0;
  diagnostics.axisError = diag[4];
  diagnostics.iterations = int(diag[5]);
  diagnostics.update = 0;
}

} // namespace duck
