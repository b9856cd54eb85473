#include "duck_model.hpp"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace duckhip {
namespace {

void require(bool ok, const char *message) {
  if (!ok)
    throw std::invalid_argument(message);
}

struct D3 {
  double x = 0, y = 0, z = 0;
};
D3 add(D3 a, D3 b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
D3 cross(D3 a, D3 b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
double dot(D3 a, D3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
D3 scale(double s, D3 a) { return {a.x * s, a.y * s, a.z * s}; }
D3 rotate(const double q[4], D3 v) {
  D3 u{q[1], q[2], q[3]};
  D3 t = add(cross(u, v), scale(q[0], v));
  return add(v, scale(2.0, cross(u, t)));
}
D3 get(const double v[3]) { return {v[0], v[1], v[2]}; }
void put(double out[3], D3 v) {
  out[0] = v.x;
  out[1] = v.y;
  out[2] = v.z;
}

void readV(std::istream &in, double v[3]) { in >> v[0] >> v[1] >> v[2]; }
void readQ(std::istream &in, double q[4]) {
  in >> q[0] >> q[1] >> q[2] >> q[3];
  double n = std::sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  if (n < 1e-15)
    throw std::runtime_error("Zero quaternion");
  for (int k = 0; k < 4; ++k)
    q[k] /= n;
}
void readUnit(std::istream &in, double v[3]) {
  readV(in, v);
  double n = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  if (n < 1e-15)
    throw std::runtime_error("Zero direction");
  double r = 1 / n;
  for (int k = 0; k < 3; ++k)
    v[k] *= r;
}

} // namespace

HostModel loadModel(const std::string &path) {
  HostModel m = parseModel(path);
  flattenModel(m);
  return m;
}

HostModel loadModelText(const std::string &text) {
  std::istringstream in(text);
  HostModel m = parseModelStream(in);
  flattenModel(m);
  return m;
}

HostModel parseModel(const std::string &path) {
  std::ifstream in(path);
  if (!in)
    throw std::runtime_error("Cannot read model: " + path);
  return parseModelStream(in);
}

HostModel parseModelStream(std::istream &in) {
  HostModel m;
  std::string header;
  int version = -1, nb = -1, nj = -1, ns = -1;
  in >> header >> version >> nb >> nj >> ns;
  if (header != "DUCK_MODEL" || (version != 1 && version != 2) || nb < 1 || nb > 10000 ||
      nj < 0 || ns < 0)
    throw std::runtime_error("Invalid model header");
  readV(in, m.gravity);
  in >> m.ground;
  m.bodies.resize(nb);
  m.joints.resize(nj);
  m.shapes.resize(ns);
  for (auto &b : m.bodies) {
    in >> b.name >> b.mass;
    readV(in, b.inertia);
    readV(in, b.x);
    readQ(in, b.q);
    readV(in, b.v);
    readV(in, b.w);
    if (b.mass < 0 || (b.mass > 0 && (b.inertia[0] <= 0 || b.inertia[1] <= 0 || b.inertia[2] <= 0)))
      throw std::runtime_error("Invalid mass/inertia");
  }
  for (auto &j : m.joints) {
    in >> j.name >> j.a >> j.b;
    readV(in, j.ra);
    readV(in, j.rb);
    readUnit(in, j.axisA);
    readUnit(in, j.axisB);
    readUnit(in, j.tangentA);
    readUnit(in, j.tangentB);
    in >> j.limited >> j.lo >> j.hi >> j.damping >> j.armature >> j.frictionloss >> j.torque >>
        j.kp >> j.target >> j.maxTorque;
    if (j.a < 0 || j.b < 0 || j.a >= nb || j.b >= nb || j.a == j.b || j.damping < 0 ||
        j.armature < 0 || j.frictionloss < 0)
      throw std::runtime_error("Invalid joint");
  }
  for (int si = 0; si < ns; ++si) {
    auto &s = m.shapes[si];
    int n = -1;
    in >> s.body >> s.type;
    readV(in, s.center);
    readQ(in, s.q);
    readV(in, s.size);
    in >> s.friction >> n;
    if (s.body < 0 || s.body >= nb || s.type < 0 || s.type > 3 || n < 0 || n > 1000000 ||
        s.friction < 0)
      throw std::runtime_error("Invalid collision shape");
    s.vertices.resize(3 * size_t(n));
    for (auto &v : s.vertices)
      in >> v;
    if (version == 2)
      in >> s.ground;
    if (s.type == 3 && n < 4)
      throw std::runtime_error("Convex mesh needs at least four vertices");
  }
  if (version == 2) {
    int count = -1;
    in >> count;
    if (count < 0 || count > 32)
      throw std::runtime_error("Invalid body collision pair count");
    for (int k = 0; k < count; ++k) {
      HostPair p;
      in >> p.a >> p.b >> p.friction;
      if (p.a < 0 || p.a >= ns || p.b <= p.a || p.b >= ns ||
          m.shapes[p.a].body == m.shapes[p.b].body || p.friction < 0 ||
          !std::isfinite(p.friction))
        throw std::runtime_error("Invalid body collision pair");
      for (auto &old : m.pairs)
        if (old.a == p.a && old.b == p.b)
          throw std::runtime_error("Duplicate body collision pair");
      m.pairs.push_back(p);
    }
  }
  if (!in)
    throw std::runtime_error("Truncated model");
  std::string extra;
  if (in >> extra)
    throw std::runtime_error("Unexpected model data");
  return m;
}

void flattenModel(HostModel &m) {
  const int nb = m.bodies.size(), nj = m.joints.size(), ns = m.shapes.size();
  // Body-frame points of boxes (8 corners) and hulls, and bounding radii
  // (solver.cpp:130-148).
  std::vector<std::vector<D3>> shapePoints(ns);
  for (int si = 0; si < ns; ++si) {
    auto &s = m.shapes[si];
    auto &pts = shapePoints[si];
    s.radius = 0;
    if (s.type == 1) {
      for (int i = 0; i < 8; ++i)
        pts.push_back(add(get(s.center), rotate(s.q, D3{(i & 1 ? 1 : -1) * s.size[0],
                                                        (i & 2 ? 1 : -1) * s.size[1],
                                                        (i & 4 ? 1 : -1) * s.size[2]})));
    } else if (s.type == 3) {
      for (size_t v = 0; v + 2 < s.vertices.size(); v += 3)
        pts.push_back(add(get(s.center),
                          rotate(s.q, D3{s.vertices[v], s.vertices[v + 1], s.vertices[v + 2]})));
    }
    for (auto p : pts)
      s.radius = std::max(s.radius, std::sqrt(dot(p, p)));
    D3 c = get(s.center);
    if (s.type == 0)
      s.radius = std::sqrt(dot(c, c)) + s.size[0];
    if (s.type == 2)
      s.radius = std::sqrt(dot(c, c)) + s.size[0] + s.size[1];
  }
  m.points.clear();
  m.colors.clear();
  m.adjacencyStart.clear();
  m.adjacency.clear();
  m.groundCapacity = 0;

  // Flattening checks (model.hpp:26-91).
  require(nb <= 32 && nj <= 32 && ns <= 32 && int(m.pairs.size()) <= 32,
          "Model capacity exceeded (32 bodies/joints/shapes)");
  require(nb > 1, "Batch needs at least one body");
  m.selfCapacity = m.pairs.size();
  if (m.ground)
    for (auto &s : m.shapes)
      if (s.ground && m.bodies[s.body].mass > 0)
        m.groundCapacity += 4;
  std::vector<int> incoming(nb, 0);
  for (auto &j : m.joints)
    require(++incoming[j.b] == 1, "A body must have at most one parent hinge");
  std::vector<bool> seen(nb);
  for (int i = 0; i < nb; ++i)
    seen[i] = incoming[i] == 0;
  m.colors.assign(nb, 0);
  for (auto &j : m.joints) {
    require(j.a < j.b, "Reset requires topological body ordering");
    require(seen[j.a], "Joint list must follow parent-before-child ordering");
    seen[j.b] = true;
    m.colors[j.b] = 1 - m.colors[j.a];
  }
  for (auto &j : m.joints)
    require(m.bodies[j.a].mass == 0 || m.bodies[j.b].mass == 0 || m.colors[j.a] != m.colors[j.b],
            "Joint graph must be bipartite");
  for (int bi = 0; bi < nb; ++bi) {
    m.adjacencyStart.push_back(m.adjacency.size());
    for (int ji = 0; ji < nj; ++ji)
      if (m.joints[ji].a == bi || m.joints[ji].b == bi)
        m.adjacency.push_back(ji);
  }
  m.adjacencyStart.push_back(m.adjacency.size());
  for (int si = 0; si < ns; ++si) {
    auto &s = m.shapes[si];
    auto &pts = shapePoints[si];
    s.offset = m.points.size() / 3;
    s.count = s.type == 0 ? 1 : (s.type == 2 ? 2 : int(pts.size()));
    D3 interior = get(s.center);
    if (!pts.empty()) {
      interior = {};
      for (auto p : pts)
        interior = add(interior, p);
      interior = scale(1 / double(pts.size()), interior);
    }
    put(s.interior, interior);
    for (auto p : pts) {
      m.points.push_back(p.x);
      m.points.push_back(p.y);
      m.points.push_back(p.z);
    }
  }
}

} // namespace duckhip
