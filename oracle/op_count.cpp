// Exact floating-point operation count of the AVBD environment step (test
// infrastructure, not product code).  The oracle's templates
// (avbd_oracle.cpp, its float64 semantics) are instantiated with a number
// type that counts every arithmetic operation it performs.  Usage:
//
//   op_count <model.duck> <steps> <iterations> <dt> <kp> <q_0> ... <q_{J-1}>
//
// resets one environment to the joint angles q, holds them as targets with
// gain kp, runs `steps` physics steps and prints the per-step averages of the
// last half of the steps (after the contacts have settled).
//
//   op_count <model.duck> <steps> <iterations> <dt> <kp> - [first]  < script
//
// reads the environment's start and controls from standard input instead:
// q_0 .. q_{J-1}, root (xyz offset, rotation vector), ground friction (< 0:
// the shapes'), mass scale, root linear velocity xyz; then per step a letter
// and its controls: `T` and J targets held with gain kp, or `M` and 3 J motor
// channels (torque, friction budget, damping per hinge).  The averages cover
// steps first .. steps - 1 (default: the last half).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace opcount {
struct Counts {
  long long add = 0, mul = 0, div = 0, sqrt = 0, trig = 0;
};
inline Counts g;
struct Counted {
  double v = 0;
  Counted() = default;
  Counted(double x) : v(x) {} // NOLINT: implicit, as a built-in real converts
  explicit operator double() const { return v; }
  explicit operator float() const { return float(v); }
  explicit operator int() const { return int(v); }
  friend Counted operator+(Counted a, Counted b) { ++g.add; return a.v + b.v; }
  friend Counted operator-(Counted a, Counted b) { ++g.add; return a.v - b.v; }
  friend Counted operator*(Counted a, Counted b) { ++g.mul; return a.v * b.v; }
  friend Counted operator/(Counted a, Counted b) { ++g.div; return a.v / b.v; }
  friend Counted operator-(Counted a) { return -a.v; }
  Counted &operator+=(Counted b) { return *this = *this + b; }
  Counted &operator-=(Counted b) { return *this = *this - b; }
  Counted &operator*=(Counted b) { return *this = *this * b; }
  Counted &operator/=(Counted b) { return *this = *this / b; }
  friend bool operator<(Counted a, Counted b) { return a.v < b.v; }
  friend bool operator>(Counted a, Counted b) { return a.v > b.v; }
  friend bool operator<=(Counted a, Counted b) { return a.v <= b.v; }
  friend bool operator>=(Counted a, Counted b) { return a.v >= b.v; }
  friend bool operator==(Counted a, Counted b) { return a.v == b.v; }
  friend bool operator!=(Counted a, Counted b) { return a.v != b.v; }
};
} // namespace opcount

// The oracle calls the <cmath> functions qualified (std::sqrt(x)); these
// overloads must be declared before its templates.
namespace std {
inline opcount::Counted sqrt(opcount::Counted a) { ++opcount::g.sqrt; return std::sqrt(a.v); }
inline opcount::Counted abs(opcount::Counted a) { return std::fabs(a.v); }
inline opcount::Counted fabs(opcount::Counted a) { return std::fabs(a.v); }
inline bool isfinite(opcount::Counted a) { return std::isfinite(a.v); }
inline bool isnan(opcount::Counted a) { return std::isnan(a.v); }
inline opcount::Counted hypot(opcount::Counted a, opcount::Counted b) {
  opcount::g.mul += 2, ++opcount::g.add, ++opcount::g.sqrt;
  return std::hypot(a.v, b.v);
}
inline opcount::Counted atan2(opcount::Counted a, opcount::Counted b) { ++opcount::g.trig; return std::atan2(a.v, b.v); }
inline opcount::Counted tan(opcount::Counted a) { ++opcount::g.trig; return std::tan(a.v); }
inline opcount::Counted sin(opcount::Counted a) { ++opcount::g.trig; return std::sin(a.v); }
inline opcount::Counted cos(opcount::Counted a) { ++opcount::g.trig; return std::cos(a.v); }
inline opcount::Counted acos(opcount::Counted a) { ++opcount::g.trig; return std::acos(a.v); }
inline opcount::Counted remainder(opcount::Counted a, opcount::Counted b) {
  ++opcount::g.trig;
  return std::remainder(a.v, b.v);
}
} // namespace std

#include "avbd_oracle.cpp"

int main(int argc, char **argv) {
  using opcount::Counted;
  if (argc < 6) {
    std::fprintf(stderr, "usage: op_count model steps iterations dt kp q...\n");
    return 2;
  }
  const int steps = std::atoi(argv[2]), iterations = std::atoi(argv[3]);
  const double dt = std::atof(argv[4]), kp = std::atof(argv[5]);
  ModelFile file = parse(argv[1]);
  HandleT<Counted> h;
  h.model = flatten<Counted>(file, dt, iterations, 0);
  h.env.initialize(h.model);
  const int nj = int(file.joints.size());
  const bool script = argc >= 7 && std::string(argv[6]) == "-";
  if (!script && argc != 6 + nj) {
    std::fprintf(stderr, "expected %d joint angles\n", nj);
    return 2;
  }
  const int first = script && argc > 7 ? std::atoi(argv[7]) : steps / 2;
  auto read = [](double &v) {
    if (std::scanf("%lf", &v) != 1) {
      std::fprintf(stderr, "op_count: truncated script\n");
      std::exit(2);
    }
  };
  std::vector<Counted> q(nj), root(6, Counted(0.0));
  double friction = -1, massScale = 1, velocity[3] = {0, 0, 0};
  for (int j = 0; j < nj; ++j) {
    double v = script ? 0 : std::atof(argv[6 + j]);
    if (script)
      read(v);
    q[j] = v;
  }
  if (script) {
    for (auto &r : root) {
      double v;
      read(v);
      r = v;
    }
    read(friction);
    read(massScale);
    for (double &v : velocity)
      read(v);
  }
  h.env.resetPose(q.data(), root.data());
  // the batch extensions of duck_reset (per-env friction, mass/inertia scale
  // of every dynamic body, root linear velocity), as the oracle applies them
  h.env.frictionOverride = Counted(friction);
  for (auto &b : h.env.bodies)
    if (b.mass > 0) {
      b.mass = b.mass * Counted(massScale);
      b.inertia = scale(Counted(massScale), b.inertia);
      b.v = {Counted(velocity[0]), Counted(velocity[1]), Counted(velocity[2])};
    }
  auto setTargets = [&](const std::vector<Counted> &target) {
    for (int j = 0; j < nj; ++j) {
      auto &jt = h.env.joints[j];
      jt.target = target[j];
      jt.kp = Counted(kp);
      jt.maxTorque = Counted(0.0);
      jt.torque = h.model.joints[j].torque;
      jt.frictionloss = h.model.joints[j].frictionloss;
      jt.damping = h.model.joints[j].damping;
    }
  };
  setTargets(q);
  opcount::Counts total;
  int counted = 0;
  for (int s = 0; s < steps; ++s) {
    if (script) {
      char kind = 0;
      if (std::scanf(" %c", &kind) != 1 || (kind != 'T' && kind != 'M')) {
        std::fprintf(stderr, "op_count: step %d needs T or M\n", s);
        return 2;
      }
      if (kind == 'T') {
        std::vector<Counted> target(nj);
        for (auto &t : target) {
          double v;
          read(v);
          t = v;
        }
        setTargets(target);
      } else {
        std::vector<Counted> motor(3 * nj);
        for (auto &m : motor) {
          double v;
          read(v);
          m = v;
        }
        Counted force[3] = {Counted(0.0), Counted(0.0), Counted(0.0)};
        h.env.setMotor(motor.data(), force);
      }
    }
    opcount::g = {};
    h.env.advance(1);
    if (s >= first) {
      total.add += opcount::g.add, total.mul += opcount::g.mul, total.div += opcount::g.div;
      total.sqrt += opcount::g.sqrt, total.trig += opcount::g.trig;
      ++counted;
    }
  }
  const double n = counted;
  std::printf("add_sub %.1f\nmul %.1f\ndiv %.1f\nsqrt %.1f\ntranscendental %.1f\n", total.add / n,
              total.mul / n, total.div / n, total.sqrt / n, total.trig / n);
  std::printf("flop_per_step %.1f\n", (total.add + total.mul + total.div + total.sqrt) / n);
  std::printf("failed %d\n", int(h.env.failed));
  return 0;
}
