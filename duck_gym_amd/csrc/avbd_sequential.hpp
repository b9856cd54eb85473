// The explicit-sequential step of the reference's independent float64 solver
// (src/solver.cpp:315-537, duck::Solver::step), one GPU thread per
// environment.
//
// It is the serial algorithm the reference runs on the host -- block
// Gauss-Seidel over the bodies in index order, the PD drive applied as an
// explicit torque in the predictor, ground contacts only -- so an environment
// has no parallel structure to spread over lanes; the batch parallelism is
// over environments (duck::Batch).  Every operation is float64 in the
// reference's order, including its std::min / std::max / std::clamp argument
// conventions, so that results track its host build to the device's
// transcendental functions.  Each environment's structs (include/duck_hip.h
// DuckSeq*) sit in one device record laid out by the host (SeqRecord); the
// thread walks them in place.  The functions are host and device code, so
// that the step's indexing can be exercised on the CPU as well.
#pragma once
#include "../../include/duck_hip.h"
#include "avbd_math.hpp"

namespace duckhip {
namespace seq {

using V = V3<double>;
using Q = Q4<double>;

// Byte offsets of an environment's arrays inside its record, written by the
// host after the header (SeqRecord) at the record's start.
struct SeqRecord {
  DuckSeqOptions options;
  int bodies, joints, shapes, points;
  int contacts;  // in: the last step's list; out: this step's
  int candidates; // entries of the candidate scratch (the largest shape's points)
  int status;
  int reserved;
  DuckSeqDiagnostics diagnostics;
  long long body, joint, shape, point, contact, old, adjacencyStart, adjacency, candidateZ,
      candidateK, torque;
};

// std::min, std::max and std::clamp as the reference's host build evaluates
// them (the first argument wins a tie; a NaN first argument passes through
// min and max).
DUCK_HD double smin(double a, double b) { return b < a ? b : a; }
DUCK_HD double smax(double a, double b) { return a < b ? b : a; }
DUCK_HD double sclamp(double v, double lo, double hi) {
  return v < lo ? lo : (hi < v ? hi : v);
}
DUCK_HD V ld3(const double *a) { return {a[0], a[1], a[2]}; }
DUCK_HD Q ld4(const double *a) { return {a[0], a[1], a[2], a[3]}; }
DUCK_HD void st3(double *a, V v) {
  a[0] = v.x;
  a[1] = v.y;
  a[2] = v.z;
}
DUCK_HD void st4(double *a, Q q) {
  a[0] = q.w;
  a[1] = q.x;
  a[2] = q.y;
  a[3] = q.z;
}
DUCK_HD double at(V v, int k) { return k == 0 ? v.x : (k == 1 ? v.y : v.z); }
DUCK_HD V unitAxis(int k, double s) {
  return {k == 0 ? s : 0.0, k == 1 ? s : 0.0, k == 2 ? s : 0.0};
}

// math.hpp:52-70 with its throws as a status (DUCK_SEQ_QUATERNION).
DUCK_HD bool normalize(Q &q, int &status) {
  const double n = sqrt(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  if (n < 1e-15) {
    status = DUCK_SEQ_QUATERNION;
    return false;
  }
  q = {q.w / n, q.x / n, q.y / n, q.z / n};
  return true;
}
DUCK_HD bool qexp(V v, Q &out, int &status) {
  const double a = norm(v), s = a < 1e-8 ? 0.5 - a * a / 48 : sin(a / 2) / a;
  out = {cos(a / 2), s * v.x, s * v.y, s * v.z};
  return normalize(out, status);
}
DUCK_HD bool qlog(Q q, V &out, int &status) {
  if (!normalize(q, status))
    return false;
  if (q.w < 0)
    q = {-q.w, -q.x, -q.y, -q.z};
  const V v{q.x, q.y, q.z};
  const double s = norm(v);
  out = v * (s < 1e-10 ? 2 : 2 * atan2(s, q.w) / s);
  return true;
}
DUCK_HD double wrapAngleSeq(double a) {
  return remainder(a, 6.283185307179586476925286766559); // 2 acos(-1.0)
}

// solver.cpp:31-36: the body inertia (or its inverse) applied in the frame
// of the step's start pose q0, the world inertia frozen over the step.
DUCK_HD V inertia(const DuckSeqBody &b, V w, bool inverse) {
  const Q q0 = ld4(b.q0);
  V local = rotate(conj(q0), w);
  local.x = local.x * (inverse ? 1 / b.inertia[0] : b.inertia[0]);
  local.y = local.y * (inverse ? 1 / b.inertia[1] : b.inertia[1]);
  local.z = local.z * (inverse ? 1 / b.inertia[2] : b.inertia[2]);
  return rotate(q0, local);
}

// math.hpp:73-80: H += k J J^T, g += f J.
DUCK_HD void stamp(double (&H)[6][6], double (&g)[6], const double (&J)[6],
                                      double force, double stiffness) {
  for (int i = 0; i < 6; ++i) {
    g[i] += J[i] * force;
    for (int j = 0; j < 6; ++j)
      H[i][j] += stiffness * J[i] * J[j];
  }
}
DUCK_HD void row(double (&J)[6], V t, V r) {
  J[0] = t.x;
  J[1] = t.y;
  J[2] = t.z;
  J[3] = r.x;
  J[4] = r.y;
  J[5] = r.z;
}

// solver.cpp:39-50: diagonal majorisation of the rotational geometric
// stiffness.
DUCK_HD void geometric(double (&H)[6][6], V r, V f) {
  const double rf = dot(r, f);
  for (int col = 0; col < 3; ++col) {
    double sum = 0;
    for (int rw = 0; rw < 3; ++rw) {
      const double a = 0.5 * (at(r, rw) * at(f, col) + at(f, rw) * at(r, col)) - (rw == col ? rf : 0);
      sum += a * a;
    }
    H[col + 3][col + 3] += sqrt(sum);
  }
}

// math.hpp:81-110: Cholesky of H and the solve of H x = -g.
DUCK_HD bool solve(const double (&H)[6][6], const double (&g)[6], double (&x)[6],
                                      int &status) {
  double L[6][6];
  for (int i = 0; i < 6; ++i)
    for (int j = 0; j < 6; ++j)
      L[i][j] = 0;
  for (int i = 0; i < 6; ++i)
    for (int j = 0; j <= i; ++j) {
      double v = H[i][j];
      for (int k = 0; k < j; ++k)
        v -= L[i][k] * L[j][k];
      if (i == j) {
        if (!(v > 0) || !__builtin_isfinite(v)) {
          status = DUCK_SEQ_HESSIAN;
          return false;
        }
        L[i][j] = sqrt(v);
      } else {
        L[i][j] = v / L[j][j];
      }
    }
  double y[6];
  for (int i = 0; i < 6; ++i) {
    y[i] = -g[i];
    for (int k = 0; k < i; ++k)
      y[i] -= L[i][k] * y[k];
    y[i] /= L[i][i];
  }
  for (int i = 5; i >= 0; --i) {
    x[i] = y[i];
    for (int k = i + 1; k < 6; ++k)
      x[i] -= L[k][i] * x[k];
    x[i] /= L[i][i];
  }
  return true;
}

// penalty bounds of the anchor (k < 3) and angular rows (solver.cpp:51-52)
DUCK_HD double minimumPenalty(int k) { return k < 3 ? 1000 : 1; }
DUCK_HD double maximumPenalty(int k) { return k < 3 ? 1e9 : 1e7; }

// One hinge evaluated at the current poses (solver.cpp:181-216): its seven
// constraint values and the world vectors its Jacobian rows are made of.
struct HingeEval {
  double C[7];
  V ra, rb, axis, axisB, t[2];
};

struct Env {
  SeqRecord *r;
  DuckSeqBody *body;
  DuckSeqJoint *joint;
  const DuckSeqShape *shape;
  const double *point;
  DuckSeqContact *contact, *old;
  const int *adjacencyStart, *adjacency;
  double *candidateZ;
  int *candidateK;
  double *torque;

  DUCK_HD explicit Env(unsigned char *base) {
    r = reinterpret_cast<SeqRecord *>(base);
    body = reinterpret_cast<DuckSeqBody *>(base + r->body);
    joint = reinterpret_cast<DuckSeqJoint *>(base + r->joint);
    shape = reinterpret_cast<const DuckSeqShape *>(base + r->shape);
    point = reinterpret_cast<const double *>(base + r->point);
    contact = reinterpret_cast<DuckSeqContact *>(base + r->contact);
    old = reinterpret_cast<DuckSeqContact *>(base + r->old);
    adjacencyStart = reinterpret_cast<const int *>(base + r->adjacencyStart);
    adjacency = reinterpret_cast<const int *>(base + r->adjacency);
    candidateZ = reinterpret_cast<double *>(base + r->candidateZ);
    candidateK = reinterpret_cast<int *>(base + r->candidateK);
    torque = reinterpret_cast<double *>(base + r->torque);
  }

  // solver.cpp:181-187
  DUCK_HD double angle(const DuckSeqJoint &j) const {
    const Q qa = ld4(body[j.a].q), qb = ld4(body[j.b].q);
    const V axis = rotate(qa, ld3(j.axis_a)), t = rotate(qa, ld3(j.tangent_a)),
            u = rotate(qb, ld3(j.tangent_b));
    return atan2(dot(axis, cross(t, u)), dot(t, u));
  }

  // solver.cpp:188-216 (the values; the rows are built from `e` by hingeRow)
  DUCK_HD void evaluate(const DuckSeqJoint &j, HingeEval &e) const {
    const DuckSeqBody &a = body[j.a], &b = body[j.b];
    const Q qa = ld4(a.q), qb = ld4(b.q);
    e.ra = rotate(qa, ld3(j.ra));
    e.rb = rotate(qb, ld3(j.rb));
    const V d = ld3(a.x) + e.ra - ld3(b.x) - e.rb;
    e.C[0] = d.x;
    e.C[1] = d.y;
    e.C[2] = d.z;
    e.axis = rotate(qa, ld3(j.axis_a));
    e.axisB = rotate(qb, ld3(j.axis_b));
    e.t[0] = rotate(qa, ld3(j.tangent_a));
    e.t[1] = cross(e.axis, e.t[0]);
    e.C[3] = dot(e.t[0], e.axisB);
    e.C[4] = dot(e.t[1], e.axisB);
    const double q = angle(j);
    e.C[5] = q - j.lo;
    e.C[6] = j.hi - q;
  }

  // Row k of the hinge's Jacobian on body a (onA) or b (solver.cpp:195-215).
  DUCK_HD static void hingeRow(const HingeEval &e, int k, bool onA, double (&J)[6]) {
    if (k < 3) {
      const V u = unitAxis(k, 1.0);
      if (onA)
        row(J, u, cross(e.ra, u));
      else
        row(J, -u, -cross(e.rb, u));
    } else if (k < 5) {
      const V t = e.t[k - 3];
      row(J, V{0, 0, 0}, onA ? cross(t, e.axisB) : cross(e.axisB, t));
    } else {
      const bool negative = (k == 5) == onA;
      row(J, V{0, 0, 0}, negative ? -e.axis : e.axis);
    }
  }

  // solver.cpp:303-314
  DUCK_HD void contactValues(const DuckSeqContact &c, V &C, V &arm) const {
    const DuckSeqBody &b = body[c.body];
    arm = rotate(ld4(b.q), ld3(c.local));
    C = ld3(b.x) + arm - ld3(c.anchor);
    C.z -= r->options.alpha * c.c0;
  }
  // solver.cpp:52-63
  DUCK_HD static V contactForce(V C, const DuckSeqContact &c) {
    V f{c.lambda[0] + c.penalty[0] * C.x, c.lambda[1] + c.penalty[1] * C.y,
        c.lambda[2] + c.penalty[2] * C.z};
    f.z = smin(f.z, 0.0);
    const double t = hypot(f.x, f.y), bound = -c.friction * f.z;
    if (t > bound && t > 0) {
      f.x *= bound / t;
      f.y *= bound / t;
    }
    return f;
  }

  // solver.cpp:216-302: up to four lowest predicted points per ground shape,
  // 5 mm apart in the ground plane, warm-started from the last step's contact
  // with the same shape and feature.
  DUCK_HD void detectContacts() {
    const DuckSeqOptions &o = r->options;
    const int previous = r->contacts;
    for (int c = 0; c < previous; ++c)
      old[c] = contact[c];
    int n = 0;
    r->contacts = 0;
    if (!o.ground)
      return;
    const double h = o.dt;
    for (int si = 0; si < r->shapes; ++si) {
      const DuckSeqShape &s = shape[si];
      if (!s.ground)
        continue;
      const DuckSeqBody &b = body[s.body];
      if (b.mass == 0)
        continue;
      const V bx = ld3(b.x), bv = ld3(b.v), bw = ld3(b.w);
      const Q bq = ld4(b.q);
      const double low =
          smin(bx.z, bx.z + h * bv.z + h * h * (o.gravity[2] + b.force[2] / b.mass));
      if (low - s.bounding_radius * (1 + h * norm(bw)) >= 0.003)
        continue;
      // the candidate points: a box's or hull's body-frame points, a
      // sphere's lowest point, a capsule's two end-cap lowest points
      V dynamic[2];
      int count = s.num_points;
      const bool staged = s.type == 1 || s.type == 3;
      if (!staged) {
        const V down = rotate(conj(bq), V{0, 0, -s.size[0]});
        const V center = ld3(s.center);
        if (s.type == 0) {
          dynamic[0] = center + down;
          count = 1;
        } else if (s.type == 2) {
          for (int i = 0; i < 2; ++i)
            dynamic[i] = center + rotate(ld4(s.q), V{0, 0, (i ? 1 : -1) * s.size[1]}) + down;
          count = 2;
        } else {
          count = 0;
        }
      }
      auto localPoint = [&](int k) { return staged ? ld3(point + 3 * (s.first_point + k)) : dynamic[k]; };
      // candidates below 3 mm, sorted by (height, index) as std::sort orders
      // the pairs: an insertion sort into the record's scratch
      int m = 0;
      for (int k = 0; k < count; ++k) {
        const V world = bx + rotate(bq, localPoint(k));
        const V velocity = bv + cross(bw, world - bx);
        const double z = smin(world.z, world.z + h * velocity.z +
                                            h * h * (o.gravity[2] + b.force[2] / b.mass));
        if (z < 0.003) {
          int at = m++;
          while (at > 0 && (z < candidateZ[at - 1] ||
                            (z == candidateZ[at - 1] && k < candidateK[at - 1]))) {
            candidateZ[at] = candidateZ[at - 1];
            candidateK[at] = candidateK[at - 1];
            --at;
          }
          candidateZ[at] = z;
          candidateK[at] = k;
        }
      }
      V chosen[4];
      int nchosen = 0;
      for (int i = 0; i < m && nchosen < 4; ++i) {
        const int k = candidateK[i];
        const V world = bx + rotate(bq, localPoint(k));
        bool duplicate = false;
        for (int c = 0; c < nchosen; ++c)
          if (hypot(chosen[c].x - world.x, chosen[c].y - world.y) < 0.005)
            duplicate = true;
        if (duplicate)
          continue;
        DuckSeqContact c{};
        c.body = s.body;
        c.shape = si;
        c.feature = k;
        st3(c.local, localPoint(k));
        c.anchor[0] = world.x;
        c.anchor[1] = world.y;
        c.anchor[2] = 0;
        c.friction = s.friction;
        for (int d = 0; d < 3; ++d)
          c.penalty[d] = 1000;
        // the cache is a map keyed by (shape, feature): the last entry wins
        for (int p = previous - 1; p >= 0; --p)
          if (old[p].shape == si && old[p].feature == k) {
            for (int d = 0; d < 3; ++d) {
              c.lambda[d] = old[p].lambda[d];
              c.penalty[d] = old[p].penalty[d];
            }
            if (old[p].stick) {
              for (int d = 0; d < 3; ++d) {
                c.local[d] = old[p].local[d];
                c.anchor[d] = old[p].anchor[d];
              }
            }
            break;
          }
        c.c0 = smin((bx + rotate(bq, ld3(c.local))).z, 0.0);
        for (int d = 0; d < 3; ++d) {
          c.lambda[d] *= o.alpha * o.gamma;
          c.penalty[d] = sclamp(c.penalty[d] * o.gamma, 1000.0, 1e9);
        }
        contact[n++] = c;
        chosen[nchosen++] = world;
      }
    }
    r->contacts = n;
  }

  // solver.cpp:363-449: one 6x6 block update of body bi; returns its update
  // norm (0 for a static body) or a negative value after a fault.
  DUCK_HD double updateBody(int bi, int &status) {
    const DuckSeqOptions &o = r->options;
    DuckSeqBody &b = body[bi];
    if (b.mass == 0)
      return 0;
    const double h = o.dt;
    double H[6][6], g[6];
    for (int i = 0; i < 6; ++i) {
      g[i] = 0;
      for (int j = 0; j < 6; ++j)
        H[i][j] = 0;
    }
    const V dx = ld3(b.x) - ld3(b.xp);
    V theta;
    if (!qlog(ld4(b.q) * conj(ld4(b.qp)), theta, status))
      return -1;
    for (int k = 0; k < 3; ++k) {
      H[k][k] = b.mass / (h * h);
      g[k] = H[k][k] * at(dx, k);
    }
    // SO(3) log Jacobian under left perturbations, frozen world inertia
    const double a = norm(theta),
                 coef = a < 1e-5 ? 1.0 / 12 + a * a / 720 : (1 - 0.5 * a / tan(0.5 * a)) / (a * a);
    V rotJ[3];
    for (int k = 0; k < 3; ++k) {
      const V e = unitAxis(k, 1.0);
      rotJ[k] = e - 0.5 * cross(theta, e) + coef * cross(theta, cross(theta, e));
    }
    for (int k = 0; k < 3; ++k) {
      g[k + 3] = dot(rotJ[k], inertia(b, theta, false)) / (h * h);
      for (int l = 0; l < 3; ++l)
        H[k + 3][l + 3] = dot(rotJ[k], inertia(b, rotJ[l], false)) / (h * h);
    }
    const Q bq = ld4(b.q);
    for (int adj = adjacencyStart[bi]; adj < adjacencyStart[bi + 1]; ++adj) {
      const DuckSeqJoint &j = joint[adjacency[adj]];
      const bool onA = bi == j.a;
      HingeEval e;
      evaluate(j, e);
      double J[6];
      for (int k = 0; k < (j.limited ? 7 : 5); ++k) {
        const double c = e.C[k] - o.alpha * (k < 5 ? j.c0[k] : smin(j.c0[k], 0.0));
        double f = j.lambda[k] + j.penalty[k] * c;
        if (k >= 5)
          f = smin(f, 0.0);
        if (k < 5 || f < 0) {
          hingeRow(e, k, onA, J);
          stamp(H, g, J, f, j.penalty[k]);
          if (k < 3) {
            geometric(H, rotate(bq, onA ? ld3(j.ra) : -ld3(j.rb)), unitAxis(k, f));
          } else if (k < 5) {
            const V ta = e.t[k - 3], ab = e.axisB;
            geometric(H, onA ? ta : ab, (onA ? ab : ta) * f);
          }
        }
      }
      hingeRow(e, 5, onA, J);
      const double delta = wrapAngleSeq(angle(j) - j.angle0),
                   stiff = j.damping / h + j.armature / (h * h),
                   force = j.damping / h * delta + j.armature / (h * h) * (delta - h * j.velocity0);
      if (stiff > 0)
        stamp(H, g, J, force, stiff);
      if (j.frictionloss > 0) {
        const double trial = j.lambda_f + j.penalty_f * delta;
        stamp(H, g, J, sclamp(trial, -j.frictionloss, j.frictionloss),
              fabs(trial) < j.frictionloss ? j.penalty_f : 0);
      }
    }
    for (int ci = 0; ci < r->contacts; ++ci) {
      const DuckSeqContact &c = contact[ci];
      if (c.body != bi)
        continue;
      V C, rr;
      contactValues(c, C, rr);
      const V f = contactForce(C, c);
      if (f.z < 0) {
        double J[6];
        for (int k = 0; k < 3; ++k) {
          const V u = unitAxis(k, 1.0);
          row(J, u, cross(rr, u));
          stamp(H, g, J, at(f, k), c.penalty[k]);
        }
        geometric(H, rotate(bq, ld3(c.local)), f);
      }
    }
    double step[6];
    if (!solve(H, g, step, status))
      return -1;
    const V tx{step[0], step[1], step[2]}, rx{step[3], step[4], step[5]};
    // std::min({1.0, ...}): the leftmost smallest
    double scale = 1.0;
    const double sx = 0.1 / smax(norm(tx), 1e-30), sr = 0.25 / smax(norm(rx), 1e-30);
    if (sx < scale)
      scale = sx;
    if (sr < scale)
      scale = sr;
    st3(b.x, ld3(b.x) + scale * tx);
    Q turn;
    if (!qexp(scale * rx, turn, status))
      return -1;
    Q q = turn * bq;
    if (!normalize(q, status))
      return -1;
    st4(b.q, q);
    return smax(norm(tx), norm(rx)) * scale;
  }

  // solver.cpp:315-537
  DUCK_HD void step() {
    int &status = r->status;
    const DuckSeqOptions &o = r->options;
    const double h = o.dt;
    DuckSeqDiagnostics &diag = r->diagnostics;
    diag = DuckSeqDiagnostics{};
    detectContacts();
    for (int ji = 0; ji < r->joints; ++ji) {
      DuckSeqJoint &j = joint[ji];
      HingeEval e;
      evaluate(j, e);
      for (int k = 0; k < 7; ++k)
        j.c0[k] = e.C[k];
      j.angle0 = angle(j);
      j.lambda_f *= o.alpha * o.gamma;
      j.penalty_f = sclamp(j.penalty_f * o.gamma, 1.0, 1e7);
      const V axis = rotate(ld4(body[j.a].q), ld3(j.axis_a));
      j.velocity0 = dot(ld3(body[j.b].w) - ld3(body[j.a].w), axis);
      for (int k = 0; k < 7; ++k) {
        j.lambda[k] *= o.alpha * o.gamma;
        j.penalty[k] = sclamp(j.penalty[k] * o.gamma, minimumPenalty(k), maximumPenalty(k));
      }
    }
    // explicit PD torques on the predictor (solver.cpp:339-347)
    for (int i = 0; i < 3 * r->bodies; ++i)
      torque[i] = 0;
    for (int ji = 0; ji < r->joints; ++ji) {
      const DuckSeqJoint &j = joint[ji];
      const V axis = rotate(ld4(body[j.a].q), ld3(j.axis_a));
      double t = j.torque + j.kp * wrapAngleSeq(j.target - j.angle0);
      if (j.max_torque > 0)
        t = sclamp(t, -j.max_torque, j.max_torque);
      st3(torque + 3 * j.b, ld3(torque + 3 * j.b) + axis * t);
      st3(torque + 3 * j.a, ld3(torque + 3 * j.a) + axis * (-t));
    }
    for (int i = 0; i < r->bodies; ++i) {
      DuckSeqBody &b = body[i];
      for (int k = 0; k < 3; ++k)
        b.x0[k] = b.x[k];
      for (int k = 0; k < 4; ++k)
        b.q0[k] = b.q[k];
      if (b.mass == 0)
        continue;
      const V g = ld3(o.gravity), force = ld3(b.force), w = ld3(b.w);
      st3(b.xp, ld3(b.x) + h * ld3(b.v) + h * h * (g + force * (1 / b.mass)));
      const V wp = w + h * inertia(b, ld3(torque + 3 * i) - cross(w, inertia(b, w, false)), true);
      Q turn;
      if (!qexp(h * wp, turn, status))
        return;
      st4(b.qp, turn * ld4(b.q));
      for (int k = 0; k < 3; ++k)
        b.x[k] = b.xp[k];
      for (int k = 0; k < 4; ++k)
        b.q[k] = b.qp[k];
    }
    for (int it = 0; it < o.iterations; ++it) {
      double maxUpdate = 0;
      for (int bi = 0; bi < r->bodies; ++bi) {
        const double update = updateBody(bi, status);
        if (status)
          return;
        maxUpdate = smax(maxUpdate, update);
      }
      // joint multipliers and stiffness ramps (solver.cpp:450-474)
      for (int ji = 0; ji < r->joints; ++ji) {
        DuckSeqJoint &j = joint[ji];
        HingeEval e;
        evaluate(j, e);
        for (int k = 0; k < (j.limited ? 7 : 5); ++k) {
          const double c = e.C[k] - o.alpha * (k < 5 ? j.c0[k] : smin(j.c0[k], 0.0));
          const double f = j.lambda[k] + j.penalty[k] * c;
          j.lambda[k] = k >= 5 ? smin(f, 0.0) : f;
          if (k < 5 || f < 0)
            j.penalty[k] = smin(j.penalty[k] + (k < 3 ? o.beta_linear : o.beta_angular) * fabs(c),
                                maximumPenalty(k));
        }
      }
      for (int ji = 0; ji < r->joints; ++ji) {
        DuckSeqJoint &j = joint[ji];
        if (j.frictionloss > 0) {
          const double delta = wrapAngleSeq(angle(j) - j.angle0);
          const double trial = j.lambda_f + j.penalty_f * delta;
          j.lambda_f = sclamp(trial, -j.frictionloss, j.frictionloss);
          if (fabs(trial) < j.frictionloss)
            j.penalty_f = smin(j.penalty_f + o.beta_angular * fabs(delta), 1e7);
        }
      }
      // contact multipliers, stick flags and ramps (solver.cpp:475-489)
      for (int ci = 0; ci < r->contacts; ++ci) {
        DuckSeqContact &c = contact[ci];
        V C, rr;
        contactValues(c, C, rr);
        const V f = contactForce(C, c);
        const double trial = hypot(c.lambda[0] + c.penalty[0] * C.x, c.lambda[1] + c.penalty[1] * C.y);
        c.stick = trial <= -c.friction * f.z && hypot(C.x, C.y) < 1e-5;
        for (int k = 0; k < 3; ++k) {
          c.lambda[k] = at(f, k);
          if (f.z < 0 && (k == 2 || trial <= -c.friction * f.z))
            c.penalty[k] = smin(c.penalty[k] + o.beta_linear * fabs(at(C, k)), 1e9);
        }
      }
      diag.update = maxUpdate;
      diag.iterations = it + 1;
      // convergence: the block updates and the constraint residuals
      // (solver.cpp:492-513)
      double error = 0;
      for (int ji = 0; ji < r->joints; ++ji) {
        const DuckSeqJoint &j = joint[ji];
        HingeEval e;
        evaluate(j, e);
        for (int k = 0; k < (j.limited ? 7 : 5); ++k) {
          const double c = e.C[k] - o.alpha * (k < 5 ? j.c0[k] : smin(j.c0[k], 0.0));
          error = smax(error, k < 5 ? fabs(c) : smax(0.0, -c));
        }
      }
      for (int ci = 0; ci < r->contacts; ++ci) {
        V C, rr;
        contactValues(contact[ci], C, rr);
        error = smax(error, smax(0.0, -C.z));
      }
      if (maxUpdate < o.tolerance && error < o.tolerance) {
        diag.converged = 1;
        break;
      }
    }
    // velocities from the pose change (solver.cpp:514-522)
    for (int i = 0; i < r->bodies; ++i) {
      DuckSeqBody &b = body[i];
      if (!(b.mass > 0))
        continue;
      const V v = (ld3(b.x) - ld3(b.x0)) * (1 / h);
      V w;
      if (!qlog(ld4(b.q) * conj(ld4(b.q0)), w, status))
        return;
      w = w * (1 / h);
      st3(b.v, v);
      st3(b.w, w);
      if (!__builtin_isfinite(norm(ld3(b.x)) + norm(v) + norm(w))) {
        status = DUCK_SEQ_NONFINITE;
        return;
      }
    }
    // diagnostics (solver.cpp:523-536)
    for (int ji = 0; ji < r->joints; ++ji) {
      HingeEval e;
      evaluate(joint[ji], e);
      for (int k = 0; k < 3; ++k)
        diag.joint_error = smax(diag.joint_error, fabs(e.C[k]));
      for (int k = 3; k < 5; ++k)
        diag.axis_error = smax(diag.axis_error, fabs(e.C[k]));
    }
    for (int ci = 0; ci < r->contacts; ++ci) {
      const DuckSeqContact &c = contact[ci];
      const DuckSeqBody &b = body[c.body];
      diag.penetration =
          smax(diag.penetration, smax(0.0, -(ld3(b.x) + rotate(ld4(b.q), ld3(c.local))).z));
    }
    diag.contacts = r->contacts;
  }
};

} // namespace seq
} // namespace duckhip
