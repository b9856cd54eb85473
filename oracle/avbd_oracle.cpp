// CPU oracle (test infrastructure): clean-room restatement of the reference
// AVBD step.  See avbd_oracle.hpp for the contract.
//
// Precision follows the reference's default build (DUCK_NATIVE_FLOAT_MATH=0,
// src/cuda/kernel.cuh:19-21): in the float instantiation a few expressions are
// evaluated in double because their literals are double (wrap, the small-angle
// exp branch, the SO(3) log-Jacobian coefficient, the geometric-stiffness
// entry, and comparisons against double thresholds).  Those spots are marked
// "[double]".  Vector division multiplies by the reciprocal, as the
// reference's Vec3 operator/ does (kernel.cuh:100).
#include "avbd_oracle.hpp"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

namespace {
thread_local std::string g_error;
thread_local long long g_flops = 0;

// ---------------------------------------------------------------- math ----
template <class R> struct V3 {
  R x = 0, y = 0, z = 0;
  R &at(int i) { return i == 0 ? x : (i == 1 ? y : z); }
  R at(int i) const { return i == 0 ? x : (i == 1 ? y : z); }
};
template <class R> struct Q4 {
  R w = 1, x = 0, y = 0, z = 0;
};
template <class R> V3<R> add(V3<R> a, V3<R> b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
template <class R> V3<R> sub(V3<R> a, V3<R> b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
template <class R> V3<R> neg(V3<R> a) { return {-a.x, -a.y, -a.z}; }
template <class R> V3<R> scale(R s, V3<R> a) { return {a.x * s, a.y * s, a.z * s}; }
// kernel.cuh:100 -- division by a scalar multiplies by its reciprocal.
template <class R> V3<R> divide(V3<R> a, R s) { return scale(R(1) / s, a); }
template <class R> R dot(V3<R> a, V3<R> b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
template <class R> V3<R> cross(V3<R> a, V3<R> b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
template <class R> R norm(V3<R> a) { return std::sqrt(dot(a, a)); }
// kernel.cuh:110-115: NaN instead of a throw on a zero direction.
template <class R> V3<R> unit(V3<R> a) {
  R n = norm(a);
  if (double(n) < 1e-15)
    return {R(NAN), R(NAN), R(NAN)};
  return divide(a, n);
}
template <class R> Q4<R> conj(Q4<R> q) { return {q.w, -q.x, -q.y, -q.z}; }
template <class R> Q4<R> mul(Q4<R> a, Q4<R> b) {
  return {a.w * b.w - a.x * b.x - a.y * b.y - a.z * b.z,
          a.w * b.x + a.x * b.w + a.y * b.z - a.z * b.y,
          a.w * b.y - a.x * b.z + a.y * b.w + a.z * b.x,
          a.w * b.z + a.x * b.y - a.y * b.x + a.z * b.w};
}
template <class R> Q4<R> normalized(Q4<R> q) {
  R n = std::sqrt(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  if (double(n) < 1e-15)
    return {R(NAN), R(NAN), R(NAN), R(NAN)};
  return {q.w / n, q.x / n, q.y / n, q.z / n};
}
// v + 2 u x (u x v + w v)  (kernel.cuh:132-135)
template <class R> V3<R> rotate(Q4<R> q, V3<R> v) {
  V3<R> u{q.x, q.y, q.z};
  return add(v, scale(R(2), cross(u, add(cross(u, v), scale(q.w, v)))));
}
// SO(3) exponential (kernel.cuh:136-145).
template <class R> Q4<R> expmap(V3<R> v) {
  R a = norm(v);
  R s;
  if (double(a) < 1e-8)
    s = R(0.5 - double(a * a / R(48))); // [double]
  else
    s = std::sin(a / R(2)) / a;
  return normalized(Q4<R>{std::cos(a / R(2)), s * v.x, s * v.y, s * v.z});
}
// SO(3) logarithm (kernel.cuh:146-153).
template <class R> V3<R> logmap(Q4<R> q) {
  q = normalized(q);
  if (q.w < 0)
    q = {-q.w, -q.x, -q.y, -q.z};
  V3<R> v{q.x, q.y, q.z};
  R s = norm(v);
  R k = double(s) < 1e-10 ? R(2) : R(2) * std::atan2(s, q.w) / s;
  return scale(k, v);
}
// remainder(a, 2 pi) evaluated in double (kernel.cuh:154-160).  [double]
template <class R> R wrap(R a) { return R(std::remainder(double(a), 2 * std::acos(-1.0))); }
template <class R> R mn(R a, R b) { return a < b ? a : b; }
template <class R> R mx(R a, R b) { return a > b ? a : b; }
template <class R> R clampv(R v, R a, R b) { return mn(mx(v, a), b); }

template <class R> struct Row6 {
  R v[6]{};
};
template <class R> Row6<R> row(V3<R> t, V3<R> r) { return {{t.x, t.y, t.z, r.x, r.y, r.z}}; }
template <class R> struct Mat6 {
  R m[6][6]{};
};
// Accumulate J^T f and k J^T J (kernel.cuh:164-176).
template <class R> void stamp(Mat6<R> &H, Row6<R> &g, const Row6<R> &J, R force, R k) {
  g_flops += 6 * 2 + 36 * 3;
  for (int i = 0; i < 6; ++i) {
    g.v[i] += J.v[i] * force;
    for (int j = 0; j < 6; ++j)
      H.m[i][j] += k * J.v[i] * J.v[j];
  }
}
// Cholesky solve of H x = -g; NaN on a non-positive pivot (kernel.cuh:177-228).
template <class R> Row6<R> cholesky(const Mat6<R> &H, const Row6<R> &g) {
  g_flops += 91 + 36 + 36;
  R L[6][6]{};
  for (int i = 0; i < 6; ++i)
    for (int j = 0; j <= i; ++j) {
      R v = H.m[i][j];
      for (int k = 0; k < j; ++k)
        v -= L[i][k] * L[j][k];
      if (i == j) {
        if (!(v > 0) || !std::isfinite(v)) {
          Row6<R> bad;
          for (auto &x : bad.v)
            x = R(NAN);
          return bad;
        }
        L[i][j] = std::sqrt(v);
      } else {
        L[i][j] = v / L[j][j];
      }
    }
  Row6<R> y, x;
  for (int i = 0; i < 6; ++i) {
    y.v[i] = -g.v[i];
    for (int k = 0; k < i; ++k)
      y.v[i] -= L[i][k] * y.v[k];
    y.v[i] /= L[i][i];
  }
  for (int i = 5; i >= 0; --i) {
    x.v[i] = y.v[i];
    for (int k = i + 1; k < 6; ++k)
      x.v[i] -= L[k][i] * x.v[k];
    x.v[i] /= L[i][i];
  }
  return x;
}
// Diagonal majorisation of the rotational geometric stiffness
// (kernel.cuh:283-301; AVBD paper Sec. 3.5).
template <class R> void geometric(Mat6<R> &H, V3<R> r, V3<R> f) {
  g_flops += 3 * 3 * 6 + 3 * 2 + 5;
  R rf = dot(r, f);
  for (int col = 0; col < 3; ++col) {
    R sum = 0;
    for (int rw = 0; rw < 3; ++rw) {
      R a = R(0.5 * double(r.at(rw) * f.at(col) + f.at(rw) * r.at(col)) -
              double(rw == col ? rf : R(0))); // [double]
      sum += a * a;
    }
    H.m[col + 3][col + 3] += std::sqrt(sum);
  }
}
template <class R> R minPenalty(int k) { return k < 3 ? R(1000) : R(1); }
template <class R> R maxPenalty(int k) { return k < 3 ? R(1e9) : R(1e7); }

// ---------------------------------------------------------- model file ----
// Parsed `.duck` v1/v2 text (src/solver.cpp:67-174), kept in double.
struct FileBody {
  std::string name;
  double mass = 0;
  V3<double> inertia, x, v, w;
  Q4<double> q;
};
struct FileJoint {
  std::string name;
  int a = 0, b = 0;
  V3<double> ra, rb, axisA, axisB, tangentA, tangentB;
  bool limited = false;
  double lo = 0, hi = 0, damping = 0, armature = 0, frictionloss = 0, torque = 0, kp = 0,
         target = 0, maxTorque = 0;
};
struct FileShape {
  int body = 0, type = 0;
  V3<double> center, size;
  Q4<double> q;
  double friction = 0.8, radius = 0;
  std::vector<V3<double>> vertices, points;
  bool ground = true;
};
struct FilePair {
  int a = 0, b = 0;
  double friction = 0;
};
struct ModelFile {
  V3<double> gravity{0, 0, -9.81};
  bool ground = false;
  std::vector<FileBody> bodies;
  std::vector<FileJoint> joints;
  std::vector<FileShape> shapes;
  std::vector<FilePair> pairs;
};

void fail(bool bad, const char *message) {
  if (bad)
    throw std::runtime_error(message);
}

V3<double> readV(std::istream &in) {
  V3<double> v;
  in >> v.x >> v.y >> v.z;
  return v;
}
Q4<double> readQ(std::istream &in) {
  Q4<double> q;
  in >> q.w >> q.x >> q.y >> q.z;
  double n = std::sqrt(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  fail(n < 1e-15, "Zero quaternion");
  return {q.w / n, q.x / n, q.y / n, q.z / n};
}
V3<double> unitOrThrow(V3<double> v) {
  double n = norm(v);
  fail(n < 1e-15, "Zero direction");
  return divide(v, n);
}

// src/solver.cpp:67-174
ModelFile parse(const std::string &path) {
  std::ifstream in(path);
  fail(!in, ("Cannot read model: " + path).c_str());
  ModelFile m;
  std::string header;
  int version = -1, nb = -1, nj = -1, ns = -1;
  in >> header >> version >> nb >> nj >> ns;
  fail(header != "DUCK_MODEL" || (version != 1 && version != 2) || nb < 1 || nb > 10000 ||
           nj < 0 || ns < 0,
       "Invalid model header");
  m.gravity = readV(in);
  in >> m.ground;
  m.bodies.resize(nb);
  m.joints.resize(nj);
  m.shapes.resize(ns);
  for (auto &b : m.bodies) {
    in >> b.name >> b.mass;
    b.inertia = readV(in);
    b.x = readV(in);
    b.q = readQ(in);
    b.v = readV(in);
    b.w = readV(in);
    fail(b.mass < 0 || (b.mass > 0 && (b.inertia.x <= 0 || b.inertia.y <= 0 || b.inertia.z <= 0)),
         "Invalid mass/inertia");
  }
  for (auto &j : m.joints) {
    in >> j.name >> j.a >> j.b;
    j.ra = readV(in);
    j.rb = readV(in);
    j.axisA = unitOrThrow(readV(in));
    j.axisB = unitOrThrow(readV(in));
    j.tangentA = unitOrThrow(readV(in));
    j.tangentB = unitOrThrow(readV(in));
    in >> j.limited >> j.lo >> j.hi >> j.damping >> j.armature >> j.frictionloss >> j.torque >>
        j.kp >> j.target >> j.maxTorque;
    fail(j.a < 0 || j.b < 0 || j.a >= nb || j.b >= nb || j.a == j.b || j.damping < 0 ||
             j.armature < 0 || j.frictionloss < 0,
         "Invalid joint");
  }
  for (auto &s : m.shapes) {
    int n = -1;
    in >> s.body >> s.type;
    s.center = readV(in);
    s.q = readQ(in);
    s.size = readV(in);
    in >> s.friction >> n;
    fail(s.body < 0 || s.body >= nb || s.type < 0 || s.type > 3 || n < 0 || n > 1000000 ||
             s.friction < 0,
         "Invalid collision shape");
    for (int k = 0; k < n; ++k)
      s.vertices.push_back(readV(in));
    if (version == 2)
      in >> s.ground;
    fail(s.type == 3 && n < 4, "Convex mesh needs at least four vertices");
    if (s.type == 1) {
      for (int i = 0; i < 8; ++i)
        s.points.push_back(add(s.center, rotate(s.q, V3<double>{(i & 1 ? 1 : -1) * s.size.x,
                                                                (i & 2 ? 1 : -1) * s.size.y,
                                                                (i & 4 ? 1 : -1) * s.size.z})));
    } else if (s.type == 3) {
      for (auto v : s.vertices)
        s.points.push_back(add(s.center, rotate(s.q, v)));
    }
    for (auto p : s.points)
      s.radius = std::max(s.radius, norm(p));
    if (s.type == 0)
      s.radius = norm(s.center) + s.size.x;
    if (s.type == 2)
      s.radius = norm(s.center) + s.size.x + s.size.y;
  }
  if (version == 2) {
    int count = -1;
    in >> count;
    fail(count < 0 || count > 32, "Invalid body collision pair count");
    for (int k = 0; k < count; ++k) {
      FilePair p;
      in >> p.a >> p.b >> p.friction;
      fail(p.a < 0 || p.a >= ns || p.b <= p.a || p.b >= ns ||
               m.shapes[p.a].body == m.shapes[p.b].body || p.friction < 0 ||
               !std::isfinite(p.friction),
           "Invalid body collision pair");
      for (auto &old : m.pairs)
        fail(old.a == p.a && old.b == p.b, "Duplicate body collision pair");
      m.pairs.push_back(p);
    }
  }
  fail(!in, "Truncated model");
  std::string extra;
  fail(bool(in >> extra), "Unexpected model data");
  return m;
}

// Angle between the joint tangents about the parent axis (kernel.cuh:725-731).
template <class R> R hingeAngle(Q4<R> qa, Q4<R> qb, V3<R> axisA, V3<R> tangentA, V3<R> tangentB) {
  V3<R> axis = rotate(qa, axisA), t = rotate(qa, tangentA), u = rotate(qb, tangentB);
  return std::atan2(dot(axis, cross(t, u)), dot(t, u));
}

// ------------------------------------------------------------ state -------
template <class R> struct Body {
  R mass = 0;
  V3<R> inertia, x, v, w, x0, xp, force;
  Q4<R> q, q0, qp;
};
template <class R> struct Joint {
  int a = 0, b = 0;
  V3<R> ra, rb, axisA, axisB, tangentA, tangentB;
  R lo = 0, hi = 0, damping = 0, armature = 0, frictionloss = 0, lambdaF = 0, penaltyF = 1,
    torque = 0, kp = 0, target = 0, maxTorque = 0;
  bool limited = false;
  R angle0 = 0, velocity0 = 0;
  R lambda[7]{}, penalty[7]{}, c0[7]{};
};
template <class R> struct Shape {
  int body = 0, type = 0, offset = 0, count = 0;
  bool ground = true;
  V3<R> center, size, interior;
  Q4<R> q;
  R friction = R(0.8), radius = 0;
};
template <class R> struct Contact {
  int body = 0, shape = 0, feature = 0, other = -1, otherShape = -1;
  V3<R> local, anchor, localB;
  V3<R> t1{1, 0, 0}, t2{0, 1, 0}, n{0, 0, 1};
  R friction = 0, c0 = 0;
  R lambda[3]{}, penalty[3]{};
  bool stick = false;
};
template <class R> struct Diag {
  R jointError = 0, axisError = 0, penetration = 0, update = 0;
  int contacts = 0, iterations = 0;
  bool converged = false;
};

// Flattened model (src/cuda/model.hpp:20-143).
template <class R> struct Model {
  std::vector<Body<R>> bodies;
  std::vector<Joint<R>> joints;
  std::vector<Shape<R>> shapes;
  std::vector<V3<R>> points;
  std::vector<FilePair> pairs;
  std::vector<int> colors, adjacencyStart, adjacency;
  R dt = 0, tolerance = 0, alpha = R(0.9), gamma = R(0.99), betaLinear = R(1e7),
    betaAngular = R(1e5);
  int iterations = 1;
  V3<R> gravity;
  bool ground = false;
  int contactCapacity = 0;
};

template <class R> V3<R> cast(V3<double> v) { return {R(v.x), R(v.y), R(v.z)}; }
template <class R> Q4<R> cast(Q4<double> q) { return {R(q.w), R(q.x), R(q.y), R(q.z)}; }

template <class R> Model<R> flatten(const ModelFile &f, double dt, int iterations, int mode) {
  Model<R> m;
  int nb = f.bodies.size();
  fail(nb < 2, "Batch needs at least one body");
  fail(nb > 32 || f.joints.size() > 32 || f.shapes.size() > 32 || f.pairs.size() > 32,
       "Model capacity exceeded (32 bodies/joints/shapes)");
  fail(mode == 1 && !f.pairs.empty(), "Body contacts require the shared CpuBatch/CUDA solver");
  int capacity = f.pairs.size();
  if (f.ground)
    for (auto &s : f.shapes)
      if (s.ground && f.bodies[s.body].mass > 0)
        capacity += 4;
  m.contactCapacity = capacity;
  for (auto &b : f.bodies) {
    Body<R> d;
    d.mass = R(b.mass);
    d.inertia = cast<R>(b.inertia);
    d.x = cast<R>(b.x);
    d.v = cast<R>(b.v);
    d.w = cast<R>(b.w);
    d.q = cast<R>(b.q);
    m.bodies.push_back(d);
  }
  // Colours by hinge-tree depth parity (model.hpp:54-91).
  m.colors.assign(nb, 0);
  std::vector<int> parents(nb, 0);
  std::vector<bool> seen(nb);
  for (auto &j : f.joints)
    fail(++parents[j.b] != 1, "A body must have at most one parent hinge");
  for (int i = 0; i < nb; ++i)
    seen[i] = parents[i] == 0;
  for (auto &j : f.joints) {
    fail(j.a >= j.b, "Reset requires topological body ordering");
    fail(!seen[j.a], "Joint list must follow parent-before-child ordering");
    seen[j.b] = true;
    m.colors[j.b] = 1 - m.colors[j.a];
    Joint<R> d;
    d.a = j.a;
    d.b = j.b;
    d.ra = cast<R>(j.ra);
    d.rb = cast<R>(j.rb);
    d.axisA = cast<R>(j.axisA);
    d.axisB = cast<R>(j.axisB);
    d.tangentA = cast<R>(j.tangentA);
    d.tangentB = cast<R>(j.tangentB);
    d.lo = R(j.lo);
    d.hi = R(j.hi);
    d.limited = j.limited;
    d.damping = R(j.damping);
    d.armature = R(j.armature);
    d.frictionloss = R(j.frictionloss);
    d.torque = R(j.torque);
    d.kp = R(j.kp);
    d.target = R(j.target);
    d.maxTorque = R(j.maxTorque);
    for (int k = 0; k < 7; ++k)
      d.penalty[k] = minPenalty<R>(k);
    m.joints.push_back(d);
  }
  for (auto &j : f.joints)
    fail(!(f.bodies[j.a].mass == 0 || f.bodies[j.b].mass == 0 || m.colors[j.a] != m.colors[j.b]),
         "Joint graph must be bipartite");
  // Body -> joint CSR in original joint order (model.hpp:92-101).
  for (int bi = 0; bi < nb; ++bi) {
    m.adjacencyStart.push_back(m.adjacency.size());
    for (int ji = 0; ji < int(f.joints.size()); ++ji)
      if (f.joints[ji].a == bi || f.joints[ji].b == bi)
        m.adjacency.push_back(ji);
  }
  m.adjacencyStart.push_back(m.adjacency.size());
  for (auto &s : f.shapes) {
    Shape<R> d;
    d.body = s.body;
    d.ground = s.ground;
    d.type = s.type;
    d.center = cast<R>(s.center);
    d.size = cast<R>(s.size);
    d.q = cast<R>(s.q);
    d.friction = R(s.friction);
    d.radius = R(s.radius);
    d.offset = m.points.size();
    d.count = s.type == 0 ? 1 : (s.type == 2 ? 2 : int(s.points.size()));
    V3<double> interior = s.center;
    if (!s.points.empty()) {
      interior = {};
      for (auto p : s.points)
        interior = add(interior, p);
      interior = divide(interior, double(s.points.size()));
    }
    d.interior = cast<R>(interior);
    for (auto p : s.points)
      m.points.push_back(cast<R>(p));
    m.shapes.push_back(d);
  }
  m.pairs = f.pairs;
  m.dt = R(dt);
  m.iterations = iterations;
  m.gravity = cast<R>(f.gravity);
  m.ground = f.ground;
  // model.hpp:141-142 for the coloured core; solver.cpp keeps 1e-7.
  m.tolerance = mode == 1 ? R(1e-7) : (std::is_same_v<R, float> ? R(1e-6) : R(1e-7));
  return m;
}

// --------------------------------------------------------- convex MPR -----
// Minkowski portal refinement (G. Snethen, "XenoCollide", Game Programming
// Gems 7), bounded as src/cuda/convex.cuh:124-217 bounds it.
template <class R> struct Support {
  V3<R> v, a, b;
};
template <class R> struct Hit {
  int status = 0; // 0 separated, 1 touching inflated shapes, -1 failure
  V3<R> normal, position;
  R depth = 0;
};
template <class R> struct ShapePose {
  const Shape<R> *shape;
  V3<R> x;
  Q4<R> q;
};

// convex.cuh:18-41: furthest vertex, ties to the lowest index.
template <class R>
V3<R> supportOf(const ShapePose<R> &sp, const std::vector<V3<R>> &points, V3<R> dir, R inflation) {
  const Shape<R> &s = *sp.shape;
  V3<R> ldir = rotate(conj(sp.q), dir), local;
  if (s.type == 0 || s.type == 2) {
    local = add(s.center, scale(s.size.x, unit(ldir)));
    if (s.type == 2) {
      V3<R> axis = rotate(s.q, V3<R>{0, 0, 1});
      local = add(local, scale(dot(axis, ldir) >= 0 ? s.size.y : -s.size.y, axis));
    }
  } else {
    int best = -1;
    R value = -INFINITY;
    for (int i = 0; i < s.count; ++i) {
      R c = dot(points[s.offset + i], ldir);
      if (c > value) {
        best = i;
        value = c;
      }
    }
    local = points[s.offset + (best < 0 ? 0 : best)];
  }
  return add(add(sp.x, rotate(sp.q, local)), scale(inflation, dir));
}

template <class R> struct Query {
  ShapePose<R> A, B;
  const std::vector<V3<R>> *points;
  R inflation;
  Support<R> operator()(V3<R> dir) const {
    Support<R> p;
    p.a = supportOf(A, *points, dir, inflation / R(2));
    p.b = supportOf(B, *points, neg(dir), inflation / R(2));
    p.v = sub(p.a, p.b);
    return p;
  }
};

template <class R> V3<R> portalNormal(const Support<R> p[4]) {
  return unit(cross(sub(p[2].v, p[1].v), sub(p[3].v, p[1].v)));
}
template <class R> void expandPortal(Support<R> p[4], const Support<R> &v) {
  V3<R> c = cross(v.v, p[0].v);
  if (dot(p[1].v, c) > 0) {
    if (dot(p[2].v, c) > 0)
      p[1] = v;
    else
      p[3] = v;
  } else if (dot(p[3].v, c) > 0) {
    p[2] = v;
  } else {
    p[1] = v;
  }
}
template <class R> R portalAdvance(const Support<R> p[4], const Support<R> &v, V3<R> d) {
  return dot(v.v, d) - mx(dot(p[1].v, d), mx(dot(p[2].v, d), dot(p[3].v, d)));
}
// Closest point of triangle abc to the origin with edge fallback
// (convex.cuh:79-104).
template <class R> V3<R> closestToOrigin(V3<R> a, V3<R> b, V3<R> c) {
  V3<R> best = a;
  R dist = dot(a, a);
  V3<R> v[3] = {a, b, c};
  for (int i = 0; i < 3; ++i) {
    V3<R> start = v[i], edge = sub(v[(i + 1) % 3], start);
    R sq = dot(edge, edge);
    V3<R> p = add(start, scale(sq > 0 ? clampv(-dot(start, edge) / sq, R(0), R(1)) : R(0), edge));
    if (dot(p, p) < dist) {
      dist = dot(p, p);
      best = p;
    }
  }
  V3<R> ab = sub(b, a), ac = sub(c, a), n = cross(ab, ac);
  R nn = dot(n, n);
  if (nn > 0) {
    V3<R> p = scale(dot(n, a) / nn, n);
    R u = dot(cross(sub(b, p), sub(c, p)), n) / nn;
    R w = dot(cross(sub(c, p), sub(a, p)), n) / nn;
    if (u >= 0 && w >= 0 && u + w <= 1 && dot(p, p) < dist)
      best = p;
  }
  return best;
}
// Barycentric contact position on the portal (convex.cuh:105-123).
template <class R> V3<R> portalPoint(const Support<R> p[4], V3<R> d) {
  R w[4] = {dot(cross(p[1].v, p[2].v), p[3].v), dot(cross(p[3].v, p[2].v), p[0].v),
            dot(cross(p[0].v, p[1].v), p[3].v), dot(cross(p[2].v, p[1].v), p[0].v)};
  R sum = w[0] + w[1] + w[2] + w[3];
  if (!(sum > 0)) {
    w[0] = 0;
    w[1] = dot(cross(p[2].v, p[3].v), d);
    w[2] = dot(cross(p[3].v, p[1].v), d);
    w[3] = dot(cross(p[1].v, p[2].v), d);
    sum = w[1] + w[2] + w[3];
  }
  if (!(sum > 0))
    return {R(NAN), R(NAN), R(NAN)};
  V3<R> pos;
  for (int i = 0; i < 4; ++i)
    pos = add(pos, scale(w[i] / (R(2) * sum), add(p[i].a, p[i].b)));
  return pos;
}

template <class R> Hit<R> mpr(const Query<R> &query, R tolerance) {
  Hit<R> hit;
  Support<R> p[4];
  const Shape<R> &sa = *query.A.shape, &sb = *query.B.shape;
  p[0].a = add(query.A.x, rotate(query.A.q, sa.interior));
  p[0].b = add(query.B.x, rotate(query.B.q, sb.interior));
  p[0].v = sub(p[0].a, p[0].b);
  R size = mx(R(0.001), sa.radius + sb.radius);
  R eps = tolerance * R(0.01);
  if (norm(p[0].v) < eps)
    p[0].v.x += eps * R(10);
  V3<R> dir = unit(neg(p[0].v));
  p[1] = query(dir);
  if (dot(p[1].v, dir) <= 0)
    return hit;
  dir = cross(p[0].v, p[1].v);
  if (norm(dir) <= eps * size) {
    hit.status = 1;
    hit.depth = norm(p[1].v);
    hit.normal = hit.depth > eps ? neg(unit(p[1].v)) : unit(p[0].v);
    hit.position = divide(add(p[1].a, p[1].b), R(2));
    return hit;
  }
  dir = unit(dir);
  p[2] = query(dir);
  if (dot(p[2].v, dir) <= 0)
    return hit;
  dir = unit(cross(sub(p[1].v, p[0].v), sub(p[2].v, p[0].v)));
  if (dot(dir, p[0].v) > 0) {
    std::swap(p[1], p[2]);
    dir = neg(dir);
  }
  // Portal discovery (<=128 candidates).
  bool discovered = false;
  for (int it = 0; it < 128; ++it) {
    if (!std::isfinite(dir.x))
      break;
    p[3] = query(dir);
    if (dot(p[3].v, dir) <= 0)
      return hit;
    if (dot(cross(p[1].v, p[3].v), p[0].v) < -eps * size * size) {
      p[2] = p[3];
    } else if (dot(cross(p[3].v, p[2].v), p[0].v) < -eps * size * size) {
      p[1] = p[3];
    } else {
      discovered = true;
      break;
    }
    dir = unit(cross(sub(p[1].v, p[0].v), sub(p[2].v, p[0].v)));
  }
  if (!discovered) {
    hit.status = -1;
    return hit;
  }
  // Does the origin lie behind the portal? (<=128 refinements)
  bool inside = false;
  for (int it = 0; it < 128; ++it) {
    dir = portalNormal(p);
    if (!std::isfinite(dir.x))
      break;
    if (dot(dir, p[1].v) >= -eps) {
      inside = true;
      break;
    }
    Support<R> s = query(dir);
    if (dot(s.v, dir) < 0 || portalAdvance(p, s, dir) <= tolerance)
      return hit;
    expandPortal(p, s);
  }
  if (!inside) {
    hit.status = -1;
    return hit;
  }
  // Penetration along the portal normal (<=256 refinements).
  for (int it = 0; it < 256; ++it) {
    dir = portalNormal(p);
    if (!std::isfinite(dir.x))
      break;
    Support<R> s = query(dir);
    if (portalAdvance(p, s, dir) <= tolerance) {
      V3<R> closest = closestToOrigin(p[1].v, p[2].v, p[3].v);
      hit.depth = norm(closest);
      hit.normal = hit.depth > eps ? neg(divide(closest, hit.depth)) : neg(dir);
      hit.position = portalPoint(p, dir);
      hit.status = std::isfinite(hit.position.x) ? 1 : -1;
      return hit;
    }
    expandPortal(p, s);
  }
  hit.status = -1;
  return hit;
}

// ------------------------------------------------------------- engine -----
template <class R> struct Env {
  const Model<R> *model = nullptr;
  int mode = 0;
  std::vector<Body<R>> bodies;
  std::vector<Joint<R>> joints;
  std::vector<Contact<R>> contacts, previous;
  std::vector<int> colors;
  int colorCount = 2;
  Diag<R> diag;
  int failed = 0;
  R frictionOverride = R(-1); // < 0: use the shape friction (reference semantics)

  // kernel.cuh:383-396
  void initialize(const Model<R> &m) {
    model = &m;
    bodies = m.bodies;
    joints = m.joints;
    contacts.clear();
    previous.clear();
    colors = m.colors;
    diag = {};
    failed = 0;
  }

  // kernel.cuh:397-420: zero velocities, offset the root, FK down the tree.
  void resetPose(const R *q, const R *root) {
    for (auto &b : bodies) {
      b.v = {};
      b.w = {};
      b.force = {};
    }
    bodies[1].x = add(bodies[1].x, V3<R>{root[0], root[1], root[2]});
    bodies[1].q = mul(expmap(V3<R>{root[3], root[4], root[5]}), bodies[1].q);
    for (size_t i = 0; i < joints.size(); ++i) {
      const auto &j = joints[i];
      const auto &oa = model->bodies[j.a], &ob = model->bodies[j.b];
      R original = hingeAngle(oa.q, ob.q, j.axisA, j.tangentA, j.tangentB);
      auto &a = bodies[j.a];
      auto &b = bodies[j.b];
      V3<R> axis = rotate(a.q, j.axisA);
      b.q = normalized(mul(mul(mul(expmap(scale(q[i] - original, axis)), a.q), conj(oa.q)), ob.q));
      b.x = sub(add(a.x, rotate(a.q, j.ra)), rotate(b.q, j.rb));
    }
  }

  R angle(const Joint<R> &j) const {
    return hingeAngle(bodies[j.a].q, bodies[j.b].q, j.axisA, j.tangentA, j.tangentB);
  }

  // Hinge rows: 3 anchor, 2 axis alignment, 2 one-sided limits
  // (kernel.cuh:732-761 / solver.cpp:188-215).  side 0 = parent, 1 = child.
  R evaluate(const Joint<R> &j, R C[7], Row6<R> JA[7], Row6<R> JB[7]) const {
    g_flops += 150;
    const auto &a = bodies[j.a], &b = bodies[j.b];
    V3<R> ra = rotate(a.q, j.ra), rb = rotate(b.q, j.rb);
    V3<R> d = sub(sub(add(a.x, ra), b.x), rb);
    for (int k = 0; k < 3; ++k) {
      V3<R> e;
      e.at(k) = 1;
      C[k] = d.at(k);
      JA[k] = row(e, cross(ra, e));
      JB[k] = row(neg(e), neg(cross(rb, e)));
    }
    V3<R> axis = rotate(a.q, j.axisA), axisB = rotate(b.q, j.axisB), t1 = rotate(a.q, j.tangentA),
          t2 = cross(axis, t1);
    for (int k = 3; k < 5; ++k) {
      V3<R> t = k == 3 ? t1 : t2;
      C[k] = dot(t, axisB);
      JA[k] = row(V3<R>{}, cross(t, axisB));
      JB[k] = row(V3<R>{}, cross(axisB, t));
    }
    R qang = angle(j);
    C[5] = qang - j.lo;
    C[6] = j.hi - qang;
    JA[5] = row(V3<R>{}, neg(axis));
    JB[5] = row(V3<R>{}, axis);
    JA[6] = row(V3<R>{}, axis);
    JB[6] = row(V3<R>{}, neg(axis));
    return qang;
  }

  // Inertia frozen at q0: R0 diag(I)^{+-1} R0^T w (kernel.cuh:275-280).
  V3<R> inertia(const Body<R> &b, V3<R> w, bool inverse) const {
    V3<R> local = rotate(conj(b.q0), w);
    for (int k = 0; k < 3; ++k)
      local.at(k) *= inverse ? R(1) / b.inertia.at(k) : b.inertia.at(k);
    return rotate(b.q0, local);
  }

  V3<R> contactWorld(const Contact<R> &c, V3<R> v) const {
    return add(add(scale(v.x, c.t1), scale(v.y, c.t2)), scale(v.z, c.n));
  }

  // Contact rows in the contact basis (kernel.cuh:805-827; solver.cpp:303-314).
  void contactRows(const Contact<R> &c, V3<R> &C, Row6<R> J[3], int bi = -1) const {
    const auto &a = bodies[c.body];
    V3<R> ra = rotate(a.q, c.local), delta = sub(add(a.x, ra), c.anchor), r = ra;
    R sign = 1;
    if (c.other >= 0) {
      const auto &b = bodies[c.other];
      V3<R> rb = rotate(b.q, c.localB);
      delta = sub(sub(add(a.x, ra), b.x), rb);
      if (bi == c.other) {
        r = rb;
        sign = -1;
      }
    }
    V3<R> basis[3] = {c.t1, c.t2, c.n};
    for (int k = 0; k < 3; ++k) {
      C.at(k) = dot(delta, basis[k]);
      V3<R> e = scale(sign, basis[k]);
      J[k] = row(e, cross(r, e));
    }
    C.z -= model->alpha * c.c0;
  }

  // Coulomb-projected contact force (kernel.cuh:304-315).
  V3<R> contactForce(V3<R> C, const Contact<R> &c) const {
    V3<R> f;
    for (int k = 0; k < 3; ++k)
      f.at(k) = c.lambda[k] + c.penalty[k] * C.at(k);
    f.z = mn(f.z, R(0));
    R t = std::hypot(f.x, f.y), bound = -c.friction * f.z;
    if (t > bound && t > 0) {
      f.x *= bound / t;
      f.y *= bound / t;
    }
    return f;
  }

  V3<R> point(const Shape<R> &s, const Body<R> &b, int k) const {
    if (s.type == 1 || s.type == 3)
      return model->points[s.offset + k];
    V3<R> down = rotate(conj(b.q), V3<R>{0, 0, -s.size.x});
    if (s.type == 0)
      return add(s.center, down);
    return add(add(s.center, rotate(s.q, V3<R>{0, 0, (k ? R(1) : R(-1)) * s.size.y})), down);
  }

  // Ground manifold + self contacts + colours (kernel.cuh:587-724; ground
  // half identical to solver.cpp:216-302).
  void detect() {
    const auto &m = *model;
    const R h = m.dt;
    previous = contacts;
    contacts.clear();
    colors = m.colors;
    colorCount = 2;
    for (int si = 0; si < int(m.shapes.size()); ++si) {
      const auto &s = m.shapes[si];
      const auto &b = bodies[s.body];
      if (!m.ground || !s.ground || b.mass == 0)
        continue;
      R low = mn(b.x.z, b.x.z + h * b.v.z + h * h * (m.gravity.z + b.force.z / b.mass));
      if (double(low - s.radius * (R(1) + h * norm(b.w))) >= .003)
        continue;
      V3<R> chosen[4];
      int n = 0;
      for (int pick = 0; pick < 4; ++pick) {
        // Lowest predicted point not within 5 mm (xy) of a chosen one; ties to
        // the lowest index (kernel.cuh:338-364).
        int best = -1;
        R lowest = INFINITY;
        for (int k = 0; k < s.count; ++k) {
          V3<R> local = point(s, b, k), world = add(b.x, rotate(b.q, local));
          V3<R> vel = add(b.v, cross(b.w, sub(world, b.x)));
          R z = mn(world.z, world.z + h * vel.z + h * h * (m.gravity.z + b.force.z / b.mass));
          if (double(z) >= .003 || z >= lowest)
            continue;
          bool duplicate = false;
          for (int c = 0; c < n; ++c)
            if (double(std::hypot(chosen[c].x - world.x, chosen[c].y - world.y)) < .005)
              duplicate = true;
          if (duplicate)
            continue;
          best = k;
          lowest = z;
        }
        if (best < 0)
          break;
        V3<R> local = point(s, b, best), world = add(b.x, rotate(b.q, local));
        Contact<R> c;
        c.body = s.body;
        c.shape = si;
        c.feature = best;
        c.local = local;
        c.anchor = {world.x, world.y, 0};
        c.friction = frictionOverride >= 0 ? frictionOverride : s.friction;
        c.penalty[0] = c.penalty[1] = c.penalty[2] = 1000;
        for (const auto &old : previous)
          if (old.other < 0 && old.shape == si && old.feature == best) {
            for (int d = 0; d < 3; ++d) {
              c.lambda[d] = old.lambda[d];
              c.penalty[d] = old.penalty[d];
            }
            if (old.stick) {
              c.local = old.local;
              c.anchor = old.anchor;
            }
            break;
          }
        c.c0 = mn(add(b.x, rotate(b.q, c.local)).z, R(0));
        for (int d = 0; d < 3; ++d) {
          c.lambda[d] *= m.alpha * m.gamma;
          c.penalty[d] = clampv(c.penalty[d] * m.gamma, R(1000), R(1e9));
        }
        if (int(contacts.size()) >= m.contactCapacity)
          failed = 1;
        else
          contacts.push_back(c);
        chosen[n++] = world;
      }
    }
    for (const auto &pair : m.pairs) {
      const auto &sa = m.shapes[pair.a], &sb = m.shapes[pair.b];
      const auto &a = bodies[sa.body], &b = bodies[sb.body];
      if (a.mass == 0 && b.mass == 0)
        continue;
      R skin = R(.003) + h * (norm(sub(a.v, b.v)) + norm(a.w) * sa.radius + norm(b.w) * sb.radius);
      if (norm(sub(a.x, b.x)) > sa.radius + sb.radius + skin)
        continue;
      Query<R> query{{&sa, a.x, a.q}, {&sb, b.x, b.q}, &m.points, skin};
      Hit<R> hit = mpr(query, mx(R(1e-8), m.tolerance * R(.1)));
      if (hit.status < 0) {
        failed = 1;
        continue;
      }
      if (hit.status == 0)
        continue;
      Contact<R> c;
      c.body = sa.body;
      c.other = sb.body;
      c.shape = pair.a;
      c.otherShape = pair.b;
      c.n = hit.normal;
      c.t1 = unit(cross(std::abs(c.n.x) < R(.8) ? V3<R>{1, 0, 0} : V3<R>{0, 1, 0}, c.n));
      c.t2 = cross(c.n, c.t1);
      R gap = skin - hit.depth;
      c.local = rotate(conj(a.q), sub(add(hit.position, scale(gap / R(2), c.n)), a.x));
      c.localB = rotate(conj(b.q), sub(sub(hit.position, scale(gap / R(2), c.n)), b.x));
      c.c0 = mn(gap, R(0));
      c.friction = R(pair.friction);
      c.penalty[0] = c.penalty[1] = c.penalty[2] = 1000;
      for (const auto &old : previous)
        if (old.shape == c.shape && old.otherShape == c.otherShape && dot(old.n, c.n) > R(.95) &&
            norm(rotate(a.q, sub(old.local, c.local))) < R(.005) &&
            norm(rotate(b.q, sub(old.localB, c.localB))) < R(.005)) {
          V3<R> f = contactWorld(old, V3<R>{old.lambda[0], old.lambda[1], old.lambda[2]});
          c.lambda[0] = dot(f, c.t1);
          c.lambda[1] = dot(f, c.t2);
          c.lambda[2] = dot(f, c.n);
          for (int d = 0; d < 3; ++d)
            c.penalty[d] = old.penalty[d];
          break;
        }
      for (int k = 0; k < 3; ++k) {
        c.lambda[k] *= m.alpha * m.gamma;
        c.penalty[k] = clampv(c.penalty[k] * m.gamma, R(1000), R(1e9));
      }
      if (int(contacts.size()) >= m.contactCapacity) {
        failed = 1;
        continue;
      }
      contacts.push_back(c);
      // A fresh colour cannot conflict with any hinge or contact neighbour
      // (kernel.cuh:717-720).
      if (a.mass > 0 && b.mass > 0 && colors[c.body] == colors[c.other])
        colors[c.other] = colorCount++;
    }
  }

  // One 6x6 block-descent update of body bi (kernel.cuh:828-936; explicit
  // mode without the implicit drive: solver.cpp:363-449).
  R updateBody(int bi) {
    const auto &m = *model;
    const R h = m.dt;
    auto &b = bodies[bi];
    if (b.mass == 0)
      return 0;
    g_flops += 400;
    Mat6<R> H;
    Row6<R> g;
    V3<R> dx = sub(b.x, b.xp), theta = logmap(mul(b.q, conj(b.qp)));
    for (int k = 0; k < 3; ++k) {
      H.m[k][k] = b.mass / (h * h);
      g.v[k] = H.m[k][k] * dx.at(k);
    }
    // SO(3) log Jacobian under left perturbation, world inertia frozen.
    R a = norm(theta);
    R coef;
    if (double(a) < 1e-5)
      coef = R(1.0 / 12 + double(a * a / R(720))); // [double]
    else
      coef = R((1 - 0.5 * double(a) / std::tan(0.5 * double(a))) / double(a * a)); // [double]
    V3<R> rotJ[3];
    for (int k = 0; k < 3; ++k) {
      V3<R> e;
      e.at(k) = 1;
      rotJ[k] = add(sub(e, scale(R(0.5), cross(theta, e))), scale(coef, cross(theta, cross(theta, e))));
    }
    for (int k = 0; k < 3; ++k) {
      g.v[k + 3] = dot(rotJ[k], inertia(b, theta, false)) / (h * h);
      for (int l = 0; l < 3; ++l)
        H.m[k + 3][l + 3] = dot(rotJ[k], inertia(b, rotJ[l], false)) / (h * h);
    }
    for (int adj = m.adjacencyStart[bi]; adj < m.adjacencyStart[bi + 1]; ++adj) {
      auto &j = joints[m.adjacency[adj]];
      R C[7];
      Row6<R> JA[7], JB[7];
      const R jointAngle = evaluate(j, C, JA, JB);
      const Row6<R> *J = bi == j.a ? JA : JB;
      for (int k = 0; k < (j.limited ? 7 : 5); ++k) {
        R c = C[k] - m.alpha * (k < 5 ? j.c0[k] : mn(j.c0[k], R(0)));
        R f = j.lambda[k] + j.penalty[k] * c;
        if (k >= 5)
          f = mn(f, R(0));
        if (k < 5 || f < 0) {
          stamp(H, g, J[k], f, j.penalty[k]);
          if (k < 3) {
            V3<R> e;
            e.at(k) = f;
            geometric(H, rotate(b.q, bi == j.a ? j.ra : neg(j.rb)), e);
          } else if (k < 5) {
            V3<R> aa = rotate(bodies[j.a].q, j.axisA), ta = rotate(bodies[j.a].q, j.tangentA);
            if (k == 4)
              ta = cross(aa, ta);
            V3<R> ab = rotate(bodies[j.b].q, j.axisB);
            geometric(H, bi == j.a ? ta : ab, scale(f, bi == j.a ? ab : ta));
          }
        }
      }
      if (mode == 0) {
        // Implicit torque-limited PD potential (kernel.cuh:893-902).
        R drive = j.kp * wrap(jointAngle - j.target) - j.torque;
        R driveStiffness = j.kp;
        if (j.maxTorque > 0) {
          if (std::abs(drive) >= j.maxTorque)
            driveStiffness = 0;
          drive = clampv(drive, -j.maxTorque, j.maxTorque);
        }
        stamp(H, g, J[5], drive, driveStiffness);
      }
      R delta = wrap(jointAngle - j.angle0), stiff = j.damping / h + j.armature / (h * h),
        force = j.damping / h * delta + j.armature / (h * h) * (delta - h * j.velocity0);
      if (stiff > 0)
        stamp(H, g, J[5], force, stiff);
      if (j.frictionloss > 0) {
        R trial = j.lambdaF + j.penaltyF * delta;
        stamp(H, g, J[5], clampv(trial, -j.frictionloss, j.frictionloss),
              std::abs(trial) < j.frictionloss ? j.penaltyF : R(0));
      }
    }
    for (const auto &c : contacts)
      if (c.body == bi || c.other == bi) {
        V3<R> C;
        Row6<R> J[3];
        contactRows(c, C, J, bi);
        V3<R> f = contactForce(C, c);
        if (f.z < 0) {
          for (int k = 0; k < 3; ++k)
            stamp(H, g, J[k], f.at(k), c.penalty[k]);
          geometric(H, rotate(b.q, bi == c.body ? c.local : c.localB),
                    scale(bi == c.body ? R(1) : R(-1), contactWorld(c, f)));
        }
      }
    Row6<R> step = cholesky(H, g);
    V3<R> tx{step.v[0], step.v[1], step.v[2]}, rx{step.v[3], step.v[4], step.v[5]};
    R s = mn(R(1), mn(R(.1) / mx(norm(tx), R(1e-30)), R(.25) / mx(norm(rx), R(1e-30))));
    b.x = add(b.x, scale(s, tx));
    b.q = normalized(mul(expmap(scale(s, rx)), b.q));
    return mx(norm(tx), norm(rx)) * s;
  }

  // One physics step (kernel.cuh:937-1095; explicit mode solver.cpp:315-537).
  void step() {
    const auto &m = *model;
    const R h = m.dt;
    if (!(h > 0) || m.iterations < 1 || m.alpha < 0 || m.alpha >= 1 || m.gamma <= 0 ||
        m.gamma >= 1) {
      failed = 1;
      return;
    }
    diag = {};
    detect();
    if (failed)
      return;
    const R ag = m.alpha * m.gamma;
    for (auto &j : joints) {
      R C[7];
      Row6<R> A[7], B[7];
      evaluate(j, j.c0, A, B);
      j.angle0 = angle(j);
      j.lambdaF *= ag;
      j.penaltyF = clampv(j.penaltyF * m.gamma, R(1), R(1e7));
      V3<R> axis = rotate(bodies[j.a].q, j.axisA);
      j.velocity0 = dot(sub(bodies[j.b].w, bodies[j.a].w), axis);
      for (int k = 0; k < 7; ++k) {
        j.lambda[k] *= ag;
        j.penalty[k] = clampv(j.penalty[k] * m.gamma, minPenalty<R>(k), maxPenalty<R>(k));
      }
      (void)C;
    }
    std::vector<V3<R>> torques(bodies.size());
    if (mode == 1) {
      // Explicit PD torque on the predictor (solver.cpp:339-347).
      for (auto &j : joints) {
        V3<R> axis = rotate(bodies[j.a].q, j.axisA);
        R t = j.torque + j.kp * wrap(j.target - j.angle0);
        if (j.maxTorque > 0)
          t = clampv(t, -j.maxTorque, j.maxTorque);
        torques[j.b] = add(torques[j.b], scale(t, axis));
        torques[j.a] = add(torques[j.a], scale(-t, axis));
      }
    }
    for (size_t i = 0; i < bodies.size(); ++i) {
      auto &b = bodies[i];
      b.x0 = b.x;
      b.q0 = b.q;
      if (b.mass == 0)
        continue;
      b.xp = add(add(b.x, scale(h, b.v)), scale(h * h, add(m.gravity, divide(b.force, b.mass))));
      V3<R> spin = neg(cross(b.w, inertia(b, b.w, false)));
      if (mode == 1)
        spin = sub(torques[i], cross(b.w, inertia(b, b.w, false)));
      V3<R> wp = add(b.w, scale(h, inertia(b, spin, true)));
      b.qp = mul(expmap(scale(h, wp)), b.q);
      b.x = b.xp;
      b.q = b.qp;
    }
    // Colour schedule: explicit mode is Gauss-Seidel in body order.
    std::vector<std::vector<int>> schedule;
    if (mode == 1) {
      for (int bi = 0; bi < int(bodies.size()); ++bi)
        schedule.push_back({bi});
    } else {
      schedule.resize(colorCount);
      for (int bi = 0; bi < int(bodies.size()); ++bi)
        schedule[colors[bi]].push_back(bi);
    }
    for (int it = 0; it < m.iterations; ++it) {
      R maxUpdate = 0;
      for (auto &group : schedule)
        for (int bi : group)
          maxUpdate = mx(maxUpdate, updateBody(bi));
      R error = 0;
      for (auto &j : joints) {
        R C[7];
        Row6<R> A[7], B[7];
        const R jointAngle = evaluate(j, C, A, B);
        for (int k = 0; k < (j.limited ? 7 : 5); ++k) {
          R c = C[k] - m.alpha * (k < 5 ? j.c0[k] : mn(j.c0[k], R(0)));
          R f = j.lambda[k] + j.penalty[k] * c;
          j.lambda[k] = k >= 5 ? mn(f, R(0)) : f;
          if (k < 5 || f < 0)
            j.penalty[k] = mn(j.penalty[k] + (k < 3 ? m.betaLinear : m.betaAngular) * std::abs(c),
                              maxPenalty<R>(k));
          error = mx(error, k < 5 ? std::abs(c) : mx(R(0), -c));
        }
        if (j.frictionloss > 0) {
          R delta = wrap(jointAngle - j.angle0);
          R trial = j.lambdaF + j.penaltyF * delta;
          j.lambdaF = clampv(trial, -j.frictionloss, j.frictionloss);
          if (std::abs(trial) < j.frictionloss)
            j.penaltyF = mn(j.penaltyF + m.betaAngular * std::abs(delta), R(1e7));
          if (mode == 0) {
            // Residual with the UPDATED multiplier (kernel.cuh:1017-1026).
            R residualTrial = j.lambdaF + j.penaltyF * wrap(jointAngle - j.angle0);
            error = mx(error, std::abs(j.lambdaF - clampv(residualTrial, -j.frictionloss,
                                                          j.frictionloss)) /
                                  j.penaltyF);
          }
        }
      }
      for (auto &c : contacts) {
        V3<R> C;
        Row6<R> J[3];
        contactRows(c, C, J);
        V3<R> f = contactForce(C, c);
        R trial = std::hypot(c.lambda[0] + c.penalty[0] * C.x, c.lambda[1] + c.penalty[1] * C.y);
        c.stick = trial <= -c.friction * f.z && double(std::hypot(C.x, C.y)) < 1e-5;
        for (int k = 0; k < 3; ++k) {
          c.lambda[k] = f.at(k);
          if (f.z < 0 && (k == 2 || trial <= -c.friction * f.z))
            c.penalty[k] = mn(c.penalty[k] + m.betaLinear * std::abs(C.at(k)), R(1e9));
        }
      }
      for (auto &c : contacts) {
        V3<R> C;
        Row6<R> J[3];
        contactRows(c, C, J);
        error = mx(error, mx(R(0), -C.z));
      }
      diag.update = maxUpdate;
      diag.iterations = it + 1;
      diag.converged = maxUpdate < m.tolerance && error < m.tolerance;
      if (diag.converged)
        break;
    }
    // Velocity recovery (kernel.cuh:1064-1073).
    for (auto &b : bodies)
      if (b.mass > 0) {
        b.v = divide(sub(b.x, b.x0), h);
        b.w = divide(logmap(mul(b.q, conj(b.q0))), h);
        if (!std::isfinite(norm(b.x) + norm(b.v) + norm(b.w))) {
          failed = 1;
          return;
        }
      }
    for (auto &j : joints) {
      R C[7];
      Row6<R> A[7], B[7];
      evaluate(j, C, A, B);
      for (int k = 0; k < 3; ++k)
        diag.jointError = mx(diag.jointError, std::abs(C[k]));
      for (int k = 3; k < 5; ++k)
        diag.axisError = mx(diag.axisError, std::abs(C[k]));
    }
    for (auto &c : contacts) {
      V3<R> C;
      Row6<R> J[3];
      contactRows(c, C, J);
      diag.penetration = mx(diag.penetration, mx(R(0), -(C.z + m.alpha * c.c0)));
    }
    diag.contacts = contacts.size();
  }

  // Substep loop with diagnostic aggregation (kernel.cuh:421-443).
  void advance(int substeps) {
    Diag<R> summary;
    summary.converged = true;
    for (int k = 0; k < substeps; ++k) {
      step();
      if (failed)
        break;
      summary.jointError = mx(summary.jointError, diag.jointError);
      summary.axisError = mx(summary.axisError, diag.axisError);
      summary.penetration = mx(summary.penetration, diag.penetration);
      summary.contacts = std::max(summary.contacts, diag.contacts);
      summary.converged = summary.converged && diag.converged;
      summary.iterations += diag.iterations;
    }
    diag = summary;
  }

  // Explicit actuator channels for one step (kernel.cuh:448-466).
  void setMotor(const R *motor, const R *force) {
    for (size_t i = 0; i < joints.size(); ++i) {
      auto &j = joints[i];
      for (int k = 0; k < 3; ++k)
        if (!std::isfinite(motor[3 * i + k]))
          failed = 1;
      if (motor[3 * i + 1] < 0 || motor[3 * i + 2] < 0)
        failed = 1;
      j.kp = 0;
      j.maxTorque = 0;
      j.torque = motor[3 * i];
      j.frictionloss = motor[3 * i + 1];
      j.damping = motor[3 * i + 2];
    }
    for (int k = 0; k < 3; ++k)
      if (!std::isfinite(force[k]))
        failed = 1;
    bodies[1].force = {force[0], force[1], force[2]};
  }

  void contactForces(R *out, bool groundOnly) const {
    std::fill(out, out + 3 * bodies.size(), R(0));
    for (const auto &c : contacts) {
      if (groundOnly && c.other >= 0)
        continue;
      V3<R> f = neg(contactWorld(c, V3<R>{c.lambda[0], c.lambda[1], c.lambda[2]}));
      for (int k = 0; k < 3; ++k) {
        out[c.body * 3 + k] += f.at(k);
        if (c.other >= 0)
          out[c.other * 3 + k] -= f.at(k);
      }
    }
  }

  void selfContactStats(R *out) const {
    out[0] = out[1] = 0;
    for (const auto &c : contacts)
      if (c.other >= 0) {
        V3<R> C;
        Row6<R> J[3];
        contactRows(c, C, J);
        R depth = mx(R(0), -(C.z + model->alpha * c.c0));
        if (c.lambda[2] < R(-1e-5) || depth > R(1e-6))
          out[0] += 1;
        out[1] = mx(out[1], depth);
      }
  }

  void contactCounts(R *out) const {
    out[0] = out[1] = 0;
    for (const auto &c : contacts)
      out[c.other < 0 ? 0 : 1] += 1;
  }

  // Recursive Newton-Euler at zero joint acceleration (kernel.cuh:504-554).
  void generalizedLoads(V3<R> rootOffset, R *out) const {
    size_t nb = bodies.size();
    std::vector<V3<R>> acc(nb), alpha(nb), force(nb), moment(nb), contact(nb), contactMoment(nb);
    const auto &root = bodies[1];
    acc[1] = cross(root.w, cross(root.w, rotate(root.q, rootOffset)));
    for (const auto &j : joints) {
      const auto &a = bodies[j.a], &b = bodies[j.b];
      V3<R> axis = rotate(a.q, j.axisA), ra = rotate(a.q, j.ra), rb = rotate(b.q, j.rb);
      R speed = dot(sub(b.w, a.w), axis);
      alpha[j.b] = add(alpha[j.a], scale(speed, cross(a.w, axis)));
      acc[j.b] = sub(sub(add(add(acc[j.a], cross(alpha[j.a], ra)), cross(a.w, cross(a.w, ra))),
                         cross(alpha[j.b], rb)),
                     cross(b.w, cross(b.w, rb)));
    }
    for (size_t i = 1; i < nb; ++i) {
      Body<R> b = bodies[i];
      b.q0 = b.q;
      force[i] = scale(b.mass, sub(acc[i], model->gravity));
      moment[i] = add(inertia(b, alpha[i], false), cross(b.w, inertia(b, b.w, false)));
    }
    for (const auto &c : contacts) {
      V3<R> f = neg(contactWorld(c, V3<R>{c.lambda[0], c.lambda[1], c.lambda[2]}));
      contact[c.body] = add(contact[c.body], f);
      contactMoment[c.body] =
          add(contactMoment[c.body], cross(rotate(bodies[c.body].q, c.local), f));
      if (c.other >= 0) {
        contact[c.other] = add(contact[c.other], neg(f));
        contactMoment[c.other] =
            add(contactMoment[c.other], cross(rotate(bodies[c.other].q, c.localB), neg(f)));
      }
    }
    for (int k = int(joints.size()) - 1; k >= 0; --k) {
      const auto &j = joints[k];
      const auto &a = bodies[j.a], &b = bodies[j.b];
      V3<R> axis = rotate(a.q, j.axisA), rb = rotate(b.q, j.rb), shift = sub(b.x, a.x);
      out[3 * k] = dot(axis, sub(moment[j.b], cross(rb, force[j.b])));
      out[3 * k + 1] = dot(axis, sub(contactMoment[j.b], cross(rb, contact[j.b]))) +
                       (j.limited ? -j.lambda[5] + j.lambda[6] : R(0));
      R motor = j.torque - j.kp * wrap(angle(j) - j.target);
      out[3 * k + 2] = j.maxTorque > 0 ? clampv(motor, -j.maxTorque, j.maxTorque) : motor;
      moment[j.a] = add(moment[j.a], add(moment[j.b], cross(shift, force[j.b])));
      force[j.a] = add(force[j.a], force[j.b]);
      contactMoment[j.a] = add(contactMoment[j.a], add(contactMoment[j.b], cross(shift, contact[j.b])));
      contact[j.a] = add(contact[j.a], contact[j.b]);
    }
  }

  // bodies[B,13], joints[J,2], diag[6] (kernel.cuh:555-575).
  void snapshot(R *bo, R *jo, R *d) const {
    for (size_t i = 0; i < bodies.size(); ++i) {
      const auto &v = bodies[i];
      R r[] = {v.x.x, v.x.y, v.x.z, v.q.w, v.q.x, v.q.y, v.q.z,
               v.v.x, v.v.y, v.v.z, v.w.x, v.w.y, v.w.z};
      std::copy(r, r + 13, bo + 13 * i);
    }
    for (size_t i = 0; i < joints.size(); ++i) {
      const auto &v = joints[i];
      jo[2 * i] = angle(v);
      jo[2 * i + 1] = dot(sub(bodies[v.b].w, bodies[v.a].w), rotate(bodies[v.a].q, v.axisA));
    }
    d[0] = diag.jointError;
    d[1] = diag.penetration;
    d[2] = R(diag.contacts);
    d[3] = R(diag.converged);
    d[4] = diag.axisError;
    d[5] = R(failed);
  }
};

// ------------------------------------------------------------- handles ----
struct Handle {
  virtual ~Handle() = default;
  bool fp64 = false;
  int nb = 0, nj = 0;
};
template <class R> struct HandleT final : Handle {
  Model<R> model;
  Env<R> env;
};

template <class F> int guarded(F &&f) {
  try {
    f();
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
    return 1;
  }
}
template <class F> int visit(void *h, F &&f) {
  auto *base = static_cast<Handle *>(h);
  return guarded([&] {
    if (base->fp64)
      f(*static_cast<HandleT<double> *>(base));
    else
      f(*static_cast<HandleT<float> *>(base));
  });
}
template <class H> using RealOf = decltype(std::declval<H>().model.dt);
} // namespace

extern "C" {
const char *oracle_last_error(void) { return g_error.c_str(); }

void *oracle_create(const char *path, double dt, int iterations, int fp64, int mode) {
  Handle *out = nullptr;
  guarded([&] {
    fail(!(dt > 0) || !std::isfinite(dt) || iterations < 1, "Invalid batch parameters");
    fail(mode != 0 && mode != 1, "Unknown oracle mode");
    ModelFile file = parse(path);
    // owned until every step has succeeded (a rejected model frees it)
    std::unique_ptr<Handle> made;
    if (fp64) {
      auto h = std::make_unique<HandleT<double>>();
      h->model = flatten<double>(file, dt, iterations, mode);
      h->env.initialize(h->model);
      h->env.mode = mode;
      made = std::move(h);
    } else {
      auto h = std::make_unique<HandleT<float>>();
      h->model = flatten<float>(file, dt, iterations, mode);
      h->env.initialize(h->model);
      h->env.mode = mode;
      made = std::move(h);
    }
    made->fp64 = fp64;
    made->nb = file.bodies.size();
    made->nj = file.joints.size();
    out = made.release();
  });
  return out;
}

void oracle_destroy(void *h) { delete static_cast<Handle *>(h); }

int oracle_dims(void *h, int *bodies, int *joints) {
  auto *b = static_cast<Handle *>(h);
  *bodies = b->nb;
  *joints = b->nj;
  return 0;
}

int oracle_reset(void *h, const double *q, const double *root) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> qs(p.nj), rs(6);
    bool finite = true;
    for (int i = 0; i < p.nj; ++i) {
      qs[i] = R(q[i]);
      finite = finite && std::isfinite(qs[i]);
    }
    for (int i = 0; i < 6; ++i) {
      rs[i] = R(root[i]);
      finite = finite && std::isfinite(rs[i]);
    }
    // Non-finite reset inputs mark the env failed (extension.cu:37-46).
    if (!finite) {
      p.env.failed = 1;
      return;
    }
    int mode = p.env.mode;
    R friction = p.env.frictionOverride;
    p.env.initialize(p.model);
    p.env.mode = mode;
    p.env.frictionOverride = friction;
    p.env.resetPose(qs.data(), rs.data());
  });
}

int oracle_set_controls(void *h, const double *target, const double *force, double kp,
                        double limit) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    for (int j = 0; j < p.nj; ++j) {
      auto &jt = p.env.joints[j];
      jt.target = R(target[j]);
      jt.kp = R(kp);
      jt.maxTorque = R(limit);
      jt.torque = p.model.joints[j].torque;
      jt.frictionloss = p.model.joints[j].frictionloss;
      jt.damping = p.model.joints[j].damping;
    }
    p.env.bodies[1].force = {R(force[0]), R(force[1]), R(force[2])};
  });
}

int oracle_set_motor(void *h, const double *motor, const double *force) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> m(3 * p.nj);
    for (int i = 0; i < 3 * p.nj; ++i)
      m[i] = R(motor[i]);
    R f[3] = {R(force[0]), R(force[1]), R(force[2])};
    p.env.setMotor(m.data(), f);
  });
}

// Per-env ground friction (a batch extension; < 0 restores shape friction).
int oracle_set_friction(void *h, double friction) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    p.env.frictionOverride = R(friction);
  });
}

// Scale every dynamic body's mass and inertia by `scale` (batch extension).
int oracle_set_mass_scale(void *h, double s) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    for (auto &b : p.env.bodies)
      if (b.mass > 0) {
        b.mass *= R(s);
        b.inertia = scale(R(s), b.inertia);
      }
  });
}

// Give every dynamic body the same linear/angular velocity (batch extension).
int oracle_set_root_velocity(void *h, const double *v, const double *w) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    for (auto &b : p.env.bodies)
      if (b.mass > 0) {
        b.v = {R(v[0]), R(v[1]), R(v[2])};
        b.w = {R(w[0]), R(w[1]), R(w[2])};
      }
  });
}

int oracle_advance(void *h, int substeps) {
  return visit(h, [&](auto &p) {
    if (!p.env.failed)
      p.env.advance(substeps);
  });
}

int oracle_detect(void *h) {
  return visit(h, [&](auto &p) { p.env.detect(); });
}

int oracle_failed(void *h) {
  int out = 0;
  visit(h, [&](auto &p) { out = p.env.failed; });
  return out;
}

int oracle_snapshot(void *h, double *bodies, double *joints, double *diag) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> b(13 * p.nb), j(2 * p.nj), d(6);
    p.env.snapshot(b.data(), j.data(), d.data());
    std::copy(b.begin(), b.end(), bodies);
    std::copy(j.begin(), j.end(), joints);
    std::copy(d.begin(), d.end(), diag);
  });
}

int oracle_set_body(void *h, int i, const double *x, const double *q, const double *v,
                    const double *w) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    fail(i < 0 || i >= p.nb, "Invalid body index");
    auto &b = p.env.bodies[i];
    b.x = {R(x[0]), R(x[1]), R(x[2])};
    b.q = {R(q[0]), R(q[1]), R(q[2]), R(q[3])};
    b.v = {R(v[0]), R(v[1]), R(v[2])};
    b.w = {R(w[0]), R(w[1]), R(w[2])};
  });
}

int oracle_contacts(void *h, int capacity, int *count, int *ints, double *reals) {
  return visit(h, [&](auto &p) {
    const auto &cs = p.env.contacts;
    *count = cs.size();
    for (int k = 0; k < int(cs.size()) && k < capacity; ++k) {
      const auto &c = cs[k];
      int *I = ints + 6 * k;
      double *Rr = reals + 26 * k;
      I[0] = c.body;
      I[1] = c.shape;
      I[2] = c.feature;
      I[3] = c.other;
      I[4] = c.otherShape;
      I[5] = c.stick;
      const std::decay_t<decltype(c.local)> *vs[] = {&c.local, &c.anchor, &c.localB,
                                                     &c.t1,    &c.t2,     &c.n};
      for (int v = 0; v < 6; ++v)
        for (int d = 0; d < 3; ++d)
          Rr[3 * v + d] = vs[v]->at(d);
      Rr[18] = c.friction;
      Rr[19] = c.c0;
      for (int d = 0; d < 3; ++d) {
        Rr[20 + d] = c.lambda[d];
        Rr[23 + d] = c.penalty[d];
      }
    }
  });
}

int oracle_colors(void *h, int *colors, int *count) {
  return visit(h, [&](auto &p) {
    for (int i = 0; i < p.nb; ++i)
      colors[i] = p.env.colors[i];
    *count = p.env.colorCount;
  });
}

int oracle_joint_state(void *h, double *out) {
  return visit(h, [&](auto &p) {
    for (int i = 0; i < p.nj; ++i) {
      const auto &j = p.env.joints[i];
      double *o = out + 31 * i;
      for (int k = 0; k < 7; ++k) {
        o[k] = j.lambda[k];
        o[7 + k] = j.penalty[k];
        o[14 + k] = j.c0[k];
      }
      double rest[] = {double(j.angle0), double(j.velocity0), double(j.lambdaF),
                       double(j.penaltyF), double(j.target), double(j.kp),
                       double(j.maxTorque), double(j.torque), double(j.frictionloss),
                       double(j.damping)};
      std::copy(rest, rest + 10, o + 21);
    }
  });
}

int oracle_contact_forces(void *h, int ground_only, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> o(3 * p.nb);
    p.env.contactForces(o.data(), ground_only != 0);
    std::copy(o.begin(), o.end(), out);
  });
}

int oracle_self_contact_stats(void *h, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    R o[2];
    p.env.selfContactStats(o);
    out[0] = o[0];
    out[1] = o[1];
  });
}

int oracle_contact_counts(void *h, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    R o[2];
    p.env.contactCounts(o);
    out[0] = o[0];
    out[1] = o[1];
  });
}

int oracle_generalized_loads(void *h, const double *offset, double *out) {
  return visit(h, [&](auto &p) {
    using R = RealOf<std::decay_t<decltype(p)>>;
    std::vector<R> o(3 * p.nj);
    p.env.generalizedLoads(V3<R>{R(offset[0]), R(offset[1]), R(offset[2])}, o.data());
    std::copy(o.begin(), o.end(), out);
  });
}

// Stand-alone MPR query on two hulls (cpu_bindings.cpp:187-246 semantics).
// poses[2][7] = xyz, wxyz.  out = status, depth, normal3, position3.
int oracle_convex_query(const double *va, int na, const double *vb, int nb,
                        const double *poses, double inflation, double tolerance, int fp64,
                        double *out) {
  return guarded([&] {
    fail(na < 4 || nb < 4, "Convex vertices must be (N>=4,3)");
    fail(!(inflation >= 0) || !std::isfinite(inflation) || !(tolerance > 0) ||
             !std::isfinite(tolerance),
         "Invalid collision tolerance/inflation");
    auto run = [&](auto tag) {
      using R = decltype(tag);
      std::vector<V3<R>> points;
      Shape<R> shapes[2];
      V3<R> xs[2];
      Q4<R> qs[2];
      for (int k = 0; k < 2; ++k) {
        const double *v = k == 0 ? va : vb;
        int n = k == 0 ? na : nb;
        auto &s = shapes[k];
        s.type = 3;
        s.offset = points.size();
        s.count = n;
        for (int i = 0; i < n; ++i) {
          for (int d = 0; d < 3; ++d)
            fail(!std::isfinite(v[3 * i + d]), "Nonfinite vertex");
          V3<R> x{R(v[3 * i]), R(v[3 * i + 1]), R(v[3 * i + 2])};
          points.push_back(x);
          s.interior = add(s.interior, divide(x, R(n)));
          s.radius = std::max(s.radius, norm(x));
        }
        const double *p = poses + 7 * k;
        for (int j = 0; j < 7; ++j)
          fail(!std::isfinite(p[j]), "Nonfinite pose");
        fail(p[3] * p[3] + p[4] * p[4] + p[5] * p[5] + p[6] * p[6] <= 1e-12, "Zero quaternion");
        xs[k] = {R(p[0]), R(p[1]), R(p[2])};
        qs[k] = normalized(Q4<R>{R(p[3]), R(p[4]), R(p[5]), R(p[6])});
      }
      Query<R> q{{&shapes[0], xs[0], qs[0]}, {&shapes[1], xs[1], qs[1]}, &points, R(inflation)};
      Hit<R> hit = mpr(q, R(tolerance));
      out[0] = hit.status;
      out[1] = hit.depth;
      for (int d = 0; d < 3; ++d) {
        out[2 + d] = hit.normal.at(d);
        out[5 + d] = hit.position.at(d);
      }
    };
    if (fp64)
      run(double{});
    else
      run(float{});
  });
}

long long oracle_flops(void) { return g_flops; }
}

// ------------------------------------------------------------ batch driver --
// The reference's CPU batch (src/cuda/cpu_bindings.cpp:20-168, CpuBatch32 and
// CpuBatch64): one model shared by `n` environments, which `workers` threads
// step with environment e on worker e mod workers; the same parameter checks
// and failure rules.  Test infrastructure and a CPU baseline, like the rest of
// this file.
namespace {
struct BatchHandle {
  virtual ~BatchHandle() = default;
  bool fp64 = false;
  int n = 0, nb = 0, nj = 0, workers = 1;
};
template <class R> struct BatchT final : BatchHandle {
  Model<R> model;
  std::vector<Env<R>> envs;
};
// cpu_bindings.cpp:76-111: worker w runs environments w, w + workers, ...
template <class F> void striped(int n, int workers, F &&work) {
  auto run = [&](int w) {
    for (int e = w; e < n; e += workers)
      work(e);
  };
  std::vector<std::thread> threads;
  for (int w = 1; w < workers; ++w)
    threads.emplace_back(run, w);
  run(0);
  for (auto &t : threads)
    t.join();
}
template <class F> int visitBatch(void *h, F &&f) {
  auto *base = static_cast<BatchHandle *>(h);
  return guarded([&] {
    if (base->fp64)
      f(*static_cast<BatchT<double> *>(base));
    else
      f(*static_cast<BatchT<float> *>(base));
  });
}
} // namespace

extern "C" {
// cpu_bindings.cpp:35-46
void *oracle_batch_create(const char *path, int n, double dt, int iterations, int fp64, int threads) {
  BatchHandle *out = nullptr;
  guarded([&] {
    fail(!(n > 0 && n <= 4096 && dt > 0 && std::isfinite(dt) && iterations > 0 && threads > 0 &&
           threads <= 64),
         "Invalid batch parameters");
    ModelFile file = parse(path);
    auto fill = [&](auto &b) {
      b.model = flatten<RealOf<std::decay_t<decltype(b)>>>(file, dt, iterations, 0);
      b.envs.resize(n);
      for (auto &env : b.envs)
        env.initialize(b.model);
    };
    std::unique_ptr<BatchHandle> made;
    if (fp64) {
      auto b = std::make_unique<BatchT<double>>();
      fill(*b);
      made = std::move(b);
    } else {
      auto b = std::make_unique<BatchT<float>>();
      fill(*b);
      made = std::move(b);
    }
    made->fp64 = fp64;
    made->n = n;
    made->nb = file.bodies.size();
    made->nj = file.joints.size();
    made->workers = std::min(n, threads);
    out = made.release();
  });
  return out;
}

void oracle_batch_destroy(void *h) { delete static_cast<BatchHandle *>(h); }

int oracle_batch_dims(void *h, int *n, int *bodies, int *joints) {
  auto *b = static_cast<BatchHandle *>(h);
  *n = b->n;
  *bodies = b->nb;
  *joints = b->nj;
  return 0;
}

// cpu_bindings.cpp:47-64: masked environments from the model state and the
// given pose; non-finite inputs mark an environment failed instead.
int oracle_batch_reset(void *h, const unsigned char *mask, const double *q, const double *root) {
  return visitBatch(h, [&](auto &b) {
    using R = RealOf<std::decay_t<decltype(b)>>;
    for (int e = 0; e < b.n; ++e) {
      if (!mask[e])
        continue;
      std::vector<R> qs(b.nj), rs(6);
      bool finite = true;
      for (int j = 0; j < b.nj; ++j) {
        qs[j] = R(q[size_t(e) * b.nj + j]);
        finite = finite && std::isfinite(q[size_t(e) * b.nj + j]);
      }
      for (int k = 0; k < 6; ++k) {
        rs[k] = R(root[size_t(e) * 6 + k]);
        finite = finite && std::isfinite(root[size_t(e) * 6 + k]);
      }
      if (!finite) {
        b.envs[e].failed = 1;
        continue;
      }
      b.envs[e].initialize(b.model);
      b.envs[e].resetPose(qs.data(), rs.data());
    }
  });
}

// cpu_bindings.cpp:65-111: targets, kp, limit and the model's torque,
// friction loss and damping on every hinge; a non-finite target or force
// fails the environment, which then does not step.
int oracle_batch_step(void *h, const double *target, const double *forces, int substeps, double kp,
                      double limit) {
  return visitBatch(h, [&](auto &b) {
    using R = RealOf<std::decay_t<decltype(b)>>;
    fail(!(substeps > 0 && kp >= 0 && std::isfinite(kp) && limit > 0 && std::isfinite(limit)),
         "Invalid controls");
    striped(b.n, b.workers, [&](int e) {
      Env<R> &s = b.envs[e];
      for (int j = 0; j < b.nj; ++j) {
        const R t = R(target[size_t(e) * b.nj + j]);
        if (!std::isfinite(t))
          s.failed = 1;
        auto &jt = s.joints[j];
        jt.target = t;
        jt.kp = R(kp);
        jt.maxTorque = R(limit);
        jt.torque = b.model.joints[j].torque;
        jt.frictionloss = b.model.joints[j].frictionloss;
        jt.damping = b.model.joints[j].damping;
      }
      const double *f = forces + size_t(e) * 3;
      for (int k = 0; k < 3; ++k)
        if (!std::isfinite(R(f[k])))
          s.failed = 1;
      if (s.failed)
        return;
      s.bodies[1].force = {R(f[0]), R(f[1]), R(f[2])};
      s.advance(substeps);
    });
  });
}

// cpu_bindings.cpp:112-125: one motor step per environment, in index order.
int oracle_batch_step_motor(void *h, const double *motor, const double *forces) {
  return visitBatch(h, [&](auto &b) {
    using R = RealOf<std::decay_t<decltype(b)>>;
    for (int e = 0; e < b.n; ++e) {
      Env<R> &s = b.envs[e];
      std::vector<R> m(3 * b.nj);
      for (int i = 0; i < 3 * b.nj; ++i)
        m[i] = R(motor[size_t(e) * 3 * b.nj + i]);
      R f[3] = {R(forces[size_t(e) * 3]), R(forces[size_t(e) * 3 + 1]), R(forces[size_t(e) * 3 + 2])};
      s.setMotor(m.data(), f);
      if (!s.failed)
        s.advance(1);
    }
  });
}

// cpu_bindings.cpp:156-162: bodies [n, B, 13], joints [n, J, 2], diag [n, 6]
int oracle_batch_state(void *h, double *bodies, double *joints, double *diag) {
  return visitBatch(h, [&](auto &b) {
    using R = RealOf<std::decay_t<decltype(b)>>;
    std::vector<R> bo(13 * b.nb), jo(2 * b.nj), d(6);
    for (int e = 0; e < b.n; ++e) {
      b.envs[e].snapshot(bo.data(), jo.data(), d.data());
      std::copy(bo.begin(), bo.end(), bodies + size_t(e) * 13 * b.nb);
      std::copy(jo.begin(), jo.end(), joints + size_t(e) * 2 * b.nj);
      std::copy(d.begin(), d.end(), diag + size_t(e) * 6);
    }
  });
}

int oracle_batch_contact_counts(void *h, double *out) {
  return visitBatch(h, [&](auto &b) {
    using R = RealOf<std::decay_t<decltype(b)>>;
    for (int e = 0; e < b.n; ++e) {
      R o[2];
      b.envs[e].contactCounts(o);
      out[2 * e] = o[0];
      out[2 * e + 1] = o[1];
    }
  });
}
}
