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
#include <cmath>
#include <cstdio>
#include <cstdlib>
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
  if (argc != 6 + nj) {
    std::fprintf(stderr, "expected %d joint angles\n", nj);
    return 2;
  }
  std::vector<Counted> q(nj), root(6, Counted(0.0));
  for (int j = 0; j < nj; ++j)
    q[j] = std::atof(argv[6 + j]);
  h.env.resetPose(q.data(), root.data());
  for (int j = 0; j < nj; ++j) {
    auto &jt = h.env.joints[j];
    jt.target = q[j];
    jt.kp = Counted(kp);
    jt.maxTorque = Counted(0.0);
    jt.torque = h.model.joints[j].torque;
    jt.frictionloss = h.model.joints[j].frictionloss;
    jt.damping = h.model.joints[j].damping;
  }
  opcount::Counts total;
  int counted = 0;
  for (int s = 0; s < steps; ++s) {
    opcount::g = {};
    h.env.advance(1);
    if (s >= steps / 2) {
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
