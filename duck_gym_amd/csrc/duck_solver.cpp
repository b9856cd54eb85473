// duck::Solver (include/duck/solver.hpp) over the C ABI of this library: a
// one-environment float64 device batch per Solver, written from and read
// back into the public members around each step.
#include "../../include/duck/solver.hpp"
#include "../../include/duck_hip.h"
#include "duck_model.hpp"

#include <hip/hip_runtime_api.h>

#include <cctype>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <sstream>
#include <unistd.h>

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

void Solver::step() {
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
    char path[] = "/tmp/duck_solver_XXXXXX";
    const int fd = mkstemp(path);
    if (fd < 0)
      throw std::runtime_error("cannot write a temporary model file");
    close(fd);
    {
      std::ofstream out(path);
      out << modelText(*this, true);
    }
    int gpu = 0;
    hip(hipGetDevice(&gpu), "hipGetDevice");
    const int code = duck_create(path, 1, options.dt, options.iterations, gpu, 64, 0, &d->handle);
    std::remove(path);
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
