// The duck C++ interface (include/duck/{math,solver}.hpp) over libduck_hip.so.
//
//   solver_api_test math          host-only checks of the math and the hinge
//                                 constraint Jacobians (tests/math_test.cpp's
//                                 invariants)
//   solver_api_test gpu MODEL     environments of a duck::Batch stepped on the
//                                 GPU: independence, reset, replay and reload
//                                 (tests/state_test.cpp's invariants)
//   solver_api_test batch MODEL   Batch::step (one launch) against each
//                                 environment stepped alone, and its outcome
//                                 when an environment throws
//   solver_api_test seqtrace MODEL N DT ITER [CONTROLS]
//                                 Solver::step (solver.cpp's explicit-
//                                 sequential step): body states and
//                                 diagnostics after each of N steps
//   solver_api_test trace MODEL N body poses after each of N steps of
//                                 Solver::stepImplicit
//   solver_api_test throughput MODEL ENVS N DT ITER KP
//                                 steps/s of Solver::step (one env) and of
//                                 Batch::step (ENVS envs), N steps each
// Prints one line per passed check; exits non-zero on the first failure.
#include "duck/solver.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>

using namespace duck;

static void check(bool ok, const char *what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    std::exit(1);
  }
  std::printf("ok %s\n", what);
}

static int math() {
  for (Vec3 v : {Vec3{0, 0, 0}, Vec3{1e-10, -2e-10, 3e-10}, Vec3{0.4, -0.2, 1.3},
                 Vec3{3.1, 0, 0}}) {
    check(norm(log(exp(v)) - v) < 1e-12, "log(exp(v)) == v");
    const Vec3 a{1, 2, 3};
    check(norm(rotate(conjugate(exp(v)), rotate(exp(v), a)) - a) < 1e-12, "rotation inverse");
    check(std::abs(norm(rotate(exp(v), a)) - norm(a)) < 1e-12, "rotation keeps length");
  }
  // the rotation vector of a product of rotations about one axis adds up
  check(norm(log(exp({0, 0, 0.3}) * exp({0, 0, 0.5})) - Vec3{0, 0, 0.8}) < 1e-14,
        "exp(a) exp(b) == exp(a + b) about one axis");
  check(std::abs(wrap(7.0) - (7.0 - 2 * std::acos(-1.0))) < 1e-15, "wrap");
  M6 H{};
  V6 x{1, -2, 3, -4, 5, -6}, g{};
  for (int i = 0; i < 6; ++i)
    for (int j = 0; j < 6; ++j)
      H[i][j] = (i == j ? 8 : 0) + 1.0 / (1 + i + j);
  for (int i = 0; i < 6; ++i)
    for (int j = 0; j < 6; ++j)
      g[i] -= H[i][j] * x[j];
  const V6 y = solve(H, g);
  double err = 0;
  for (int i = 0; i < 6; ++i)
    err = std::max(err, std::abs(y[i] - x[i]));
  check(err < 1e-12, "solve(H, g) = -H^-1 g");
  bool threw = false;
  try {
    solve(M6{}, V6{});
  } catch (const std::runtime_error &) {
    threw = true;
  }
  check(threw, "singular system rejected");
  M6 S{};
  V6 gs{};
  stamp(S, gs, row({1, 2, 3}, {4, 5, 6}), 0.5, 2.0);
  check(S[1][2] == 2.0 * 2 * 3 && gs[5] == 3.0, "stamp");

  // Hinge rows against central differences of C, for body rotations applied
  // in the world frame (q <- exp(d) q).  The anchor and axis rows (0-4) are
  // exact everywhere; the limit rows' +-axis Jacobian is exact where the two
  // hinge axes coincide, so they are checked on an aligned hinge.
  auto worstDifference = [](Solver &sim, const Joint &j, int rows) {
    std::array<double, 7> C{};
    std::array<V6, 7> JA{}, JB{};
    sim.evaluateJoint(j, C, JA, JB);
    double worst = 0;
    for (int body = 0; body < 2; ++body)
      for (int dof = 0; dof < 6; ++dof) {
        const Body saved = sim.bodies[body];
        std::array<double, 7> plus{}, minus{};
        std::array<V6, 7> ja{}, jb{};
        for (int s = -1; s <= 1; s += 2) {
          Vec3 d{};
          d[dof % 3] = 1e-6 * s;
          if (dof < 3)
            sim.bodies[body].x = saved.x + d;
          else
            sim.bodies[body].q = exp(d) * saved.q;
          sim.evaluateJoint(j, s > 0 ? plus : minus, ja, jb);
          sim.bodies[body] = saved;
        }
        for (int k = 0; k < rows; ++k)
          worst = std::max(worst, std::abs((plus[k] - minus[k]) / 2e-6 -
                                           (body == 0 ? JA : JB)[k][dof]));
      }
    return worst;
  };
  Solver sim;
  sim.bodies.resize(2);
  sim.bodies[0].x = {0.1, 0.2, 0.3};
  sim.bodies[1].x = {-0.2, 0.3, 0.4};
  sim.bodies[0].q = exp({0.2, -0.3, 0.1});
  sim.bodies[1].q = exp({-0.4, 0.1, 0.2});
  Joint j;
  j.a = 0;
  j.b = 1;
  j.ra = {0.03, -0.02, 0.07};
  j.rb = {-0.01, 0.05, 0.03};
  j.axisA = {0, 0, 1};
  j.axisB = {0, 1, 0};
  j.tangentA = {1, 0, 0};
  j.tangentB = {1, 0, 0};
  j.lo = -0.5;
  j.hi = 0.7;
  check(worstDifference(sim, j, 5) < 1e-8, "anchor and axis Jacobians match central differences");
  // aligned: b is a turned 0.3 rad about the hinge axis
  j.axisB = j.axisA;
  const Vec3 axisWorld = rotate(sim.bodies[0].q, j.axisA);
  sim.bodies[1].q = exp(axisWorld * 0.3) * sim.bodies[0].q;
  check(std::abs(sim.angle(j) - 0.3) < 1e-14, "hinge angle");
  check(worstDifference(sim, j, 7) < 1e-8, "all seven Jacobians on an aligned hinge");
  std::array<double, 7> C{};
  std::array<V6, 7> JA{}, JB{};
  sim.evaluateJoint(j, C, JA, JB);
  check(std::abs(C[5] - 0.8) < 1e-14 && std::abs(C[6] - 0.4) < 1e-14, "limit rows");
  // The anchor rows bit for bit: solver.cpp:192 evaluates a.x + ra - b.x - rb
  // left to right.  Over random poses, the grouping (a.x + ra) - (b.x + rb)
  // rounds differently in some component, so this check tells them apart.
  bool groupingDiffers = false;
  unsigned seed = 12345;
  auto uniform = [&seed]() {
    seed = seed * 1664525u + 1013904223u;
    return (seed >> 8) * (1.0 / 16777216.0) - 0.5;
  };
  for (int trial = 0; trial < 200; ++trial) {
    sim.bodies[0].x = {uniform(), uniform(), uniform()};
    sim.bodies[1].x = {uniform(), uniform(), uniform()};
    sim.bodies[0].q = exp({uniform(), uniform(), uniform()});
    sim.bodies[1].q = exp({uniform(), uniform(), uniform()});
    sim.evaluateJoint(j, C, JA, JB);
    const Vec3 ra = rotate(sim.bodies[0].q, j.ra), rb = rotate(sim.bodies[1].q, j.rb);
    for (int k = 0; k < 3; ++k) {
      const double ordered = sim.bodies[0].x[k] + ra[k] - sim.bodies[1].x[k] - rb[k];
      const double grouped = (sim.bodies[0].x[k] + ra[k]) - (sim.bodies[1].x[k] + rb[k]);
      check(C[k] == ordered, "anchor rows in solver.cpp's operation order");
      groupingDiffers = groupingDiffers || grouped != ordered;
    }
  }
  check(groupingDiffers, "the anchor-row check distinguishes the two groupings");
  std::printf("math checks passed\n");
  return 0;
}

static double distance(const Body &a, const Body &b) { return norm(a.x - b.x); }

static int gpu(const char *model) {
  Solver original;
  original.load(model);
  original.options.dt = 0.005;
  original.options.iterations = 10;
  check(original.bodies.size() >= 2 && original.joints.size() >= 1, "model loaded");
  original.options.dt = 0.001; // the explicit drive is stable at 1 ms
  Batch batch(original, 3);
  batch.environments[1].bodies[1].v.x = 0.1;
  for (int i = 0; i < 50; ++i)
    batch.step();
  auto &env = batch.environments;
  check(distance(env[0].bodies[1], env[2].bodies[1]) == 0, "identical environments agree");
  check(distance(env[0].bodies[1], env[1].bodies[1]) > 1e-7, "a perturbed environment differs");
  check(distance(env[0].bodies[1], original.bodies[1]) > 1e-6, "the environments moved");
  const Body reference = env[2].bodies[1];
  const auto referenceJoints = env[2].joints;
  batch.reset(0);
  check(distance(env[0].bodies[1], original.bodies[1]) == 0, "reset restores the file state");
  check(distance(env[2].bodies[1], reference) == 0, "reset leaves the others");
  for (int i = 0; i < 50; ++i)
    env[0].step();
  check(distance(env[0].bodies[1], reference) == 0 &&
            norm(env[0].bodies[1].v - reference.v) == 0,
        "a reset environment replays bit for bit");
  check(env[0].joints[0].lambda == referenceJoints[0].lambda, "replayed multipliers agree");
  env[0].load(model);
  bool zero = true;
  for (auto &jt : env[0].joints)
    for (double l : jt.lambda)
      zero = zero && l == 0;
  check(zero, "reload clears the multipliers");
  bool rejected = false;
  try {
    Batch invalid(original, 0);
  } catch (const std::exception &) {
    rejected = true;
  }
  check(rejected, "an empty batch is rejected");
  // options the implicit step does not run are refused, not ignored
  Solver changed = original;
  changed.options.alpha = 0.5;
  rejected = false;
  try {
    changed.stepImplicit();
  } catch (const std::invalid_argument &) {
    rejected = true;
  }
  check(rejected, "options the implicit step does not run are rejected");
  changed.step();
  check(changed.diagnostics.iterations > 0, "the sequential step runs other AL constants");
  changed.options.alpha = 1.5;
  rejected = false;
  try {
    changed.step();
  } catch (const std::runtime_error &e) {
    rejected = std::string(e.what()) == "Invalid solver options";
  }
  check(rejected, "invalid options rejected as solver.cpp rejects them");
  std::printf("gpu checks passed: %s\n", model);
  return 0;
}

// Bitwise equality (a NaN equals its own bits).
static bool eq(double a, double b) { return std::memcmp(&a, &b, sizeof a) == 0; }
static bool eq(Vec3 a, Vec3 b) { return eq(a.x, b.x) && eq(a.y, b.y) && eq(a.z, b.z); }
static bool eq(Quat a, Quat b) { return eq(a.w, b.w) && eq(a.x, b.x) && eq(a.y, b.y) && eq(a.z, b.z); }
template <size_t N> static bool eq(const std::array<double, N> &a, const std::array<double, N> &b) {
  for (size_t i = 0; i < N; ++i)
    if (!eq(a[i], b[i]))
      return false;
  return true;
}

// Every field a step writes, bit for bit.
static bool same(const Solver &a, const Solver &b) {
  for (size_t i = 0; i < a.bodies.size(); ++i) {
    const Body &x = a.bodies[i], &y = b.bodies[i];
    if (!eq(x.x, y.x) || !eq(x.v, y.v) || !eq(x.w, y.w) || !eq(x.q, y.q) || !eq(x.x0, y.x0) ||
        !eq(x.xp, y.xp) || !eq(x.q0, y.q0) || !eq(x.qp, y.qp))
      return false;
  }
  for (size_t i = 0; i < a.joints.size(); ++i) {
    const Joint &x = a.joints[i], &y = b.joints[i];
    if (!eq(x.lambda, y.lambda) || !eq(x.penalty, y.penalty) || !eq(x.c0, y.c0) ||
        !eq(x.angle0, y.angle0) || !eq(x.velocity0, y.velocity0) || !eq(x.lambdaF, y.lambdaF) ||
        !eq(x.penaltyF, y.penaltyF))
      return false;
  }
  if (a.contacts.size() != b.contacts.size())
    return false;
  for (size_t i = 0; i < a.contacts.size(); ++i) {
    const Contact &x = a.contacts[i], &y = b.contacts[i];
    if (x.body != y.body || x.shape != y.shape || x.feature != y.feature || x.stick != y.stick ||
        !eq(x.lambda, y.lambda) || !eq(x.penalty, y.penalty) || !eq(x.c0, y.c0) ||
        !eq(x.local, y.local) || !eq(x.anchor, y.anchor))
      return false;
  }
  const Diagnostics &p = a.diagnostics, &q = b.diagnostics;
  return eq(p.jointError, q.jointError) && eq(p.axisError, q.axisError) &&
         eq(p.penetration, q.penetration) && eq(p.update, q.update) && p.contacts == q.contacts &&
         p.iterations == q.iterations && p.converged == q.converged;
}

// Batch::step runs every environment in one launch: each ends as it would
// stepped alone, and when one throws the outcome is that of stepping them in
// order (the reference's loop): those before it stepped, it left as its step
// left it, those after it untouched.
static int batch(const char *model) {
  Solver proto;
  proto.load(model);
  proto.options.dt = 0.001;
  proto.options.iterations = 10;
  Batch all(proto, 5);
  for (int i = 0; i < 5; ++i) {
    all.environments[i].bodies[1].v.y = 0.02 * i;
    for (auto &j : all.environments[i].joints)
      j.target += 0.01 * i;
  }
  std::vector<Solver> alone = all.environments;
  for (int s = 0; s < 20; ++s) {
    all.step();
    for (auto &env : alone)
      env.step();
  }
  bool equal = true;
  for (int i = 0; i < 5; ++i)
    equal = equal && same(all.environments[i], alone[i]);
  check(equal, "Batch::step equals each environment stepped alone, bit for bit");
  check(!same(all.environments[0], all.environments[1]), "the environments differ");
  {
    // a batch past the LDS-staged kernel's size takes the device-memory
    // kernel: the same operations, so the same bits
    Batch big(proto, 80);
    for (int i = 0; i < 80; ++i) {
      big.environments[i].bodies[1].v.y = 0.02 * (i % 5);
      for (auto &j : big.environments[i].joints)
        j.target += 0.01 * (i % 5);
    }
    for (int s = 0; s < 20; ++s)
      big.step();
    bool bigEqual = true;
    for (int i = 0; i < 80; ++i)
      bigEqual = bigEqual && same(big.environments[i], alone[i % 5]);
    check(bigEqual, "an 80-environment Batch::step equals the 5-environment one, bit for bit");
  }

  auto outcome = [&](const char *what, auto &&spoil) {
    std::vector<Solver> before = all.environments;
    spoil(all.environments[2]);
    std::vector<Solver> spoiled = all.environments;
    std::string message;
    try {
      all.step();
    } catch (const std::runtime_error &e) {
      message = e.what();
    }
    std::vector<Solver> expect = spoiled;
    std::string expected;
    for (int i = 0; i < 5; ++i) {
      try {
        expect[i].step();
      } catch (const std::runtime_error &e) {
        expected = e.what();
        break;
      }
    }
    bool ok = !message.empty() && message == expected;
    for (int i = 0; i < 5; ++i)
      ok = ok && same(all.environments[i], expect[i]);
    ok = ok && same(all.environments[3], spoiled[3]) && same(all.environments[4], spoiled[4]);
    std::printf("%s: %s\n", what, message.c_str());
    check(ok, what);
    all.environments = before;
  };
  outcome("a body-contact pair in environment 2 stops the batch there", [](Solver &s) {
    s.collisionPairs.push_back(CollisionPair{0, 1, 0.5});
  });
  outcome("invalid options in environment 2 stop the batch there",
          [](Solver &s) { s.options.gamma = 1.0; });
  outcome("a numerical fault in environment 2 is thrown after it, the rest untouched",
          [](Solver &s) { s.bodies[1].v.x = std::nan(""); });
  std::printf("batch checks passed: %s\n", model);
  return 0;
}

// Solver::step of one environment: STEPS steps at DT and ITER iterations,
// with the file's controls or, from CONTROLS, J hinge targets, kp, the torque
// limit and the root force (x, y, z).  Prints after every step one line per
// body, "s b x y z qw qx qy qz vx vy vz wx wy wz", and one diagnostics line,
// "d s jointError axisError penetration update contacts iterations converged".
static int seqtrace(const char *model, int steps, double dt, int iterations,
                    const char *controls) {
  Solver sim;
  sim.load(model);
  sim.options.dt = dt;
  sim.options.iterations = iterations;
  if (controls) {
    std::ifstream in(controls);
    for (auto &j : sim.joints)
      in >> j.target;
    double kp = 0, limit = 0;
    in >> kp >> limit >> sim.bodies.at(1).force.x >> sim.bodies[1].force.y >>
        sim.bodies[1].force.z;
    if (!in)
      throw std::runtime_error("truncated controls file");
    for (auto &j : sim.joints) {
      j.kp = kp;
      j.maxTorque = limit;
    }
  }
  for (int s = 1; s <= steps; ++s) {
    sim.step();
    for (size_t b = 0; b < sim.bodies.size(); ++b) {
      const Body &x = sim.bodies[b];
      std::printf("%d %zu %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g "
                  "%.17g %.17g\n",
                  s, b, x.x.x, x.x.y, x.x.z, x.q.w, x.q.x, x.q.y, x.q.z, x.v.x, x.v.y, x.v.z, x.w.x,
                  x.w.y, x.w.z);
    }
    const Diagnostics &d = sim.diagnostics;
    std::printf("d %d %.17g %.17g %.17g %.17g %d %d %d\n", s, d.jointError, d.axisError,
                d.penetration, d.update, d.contacts, d.iterations, d.converged ? 1 : 0);
  }
  return 0;
}

// Throughput of Solver::step and duck::Batch::step (solver.cpp's step on the
// GPU): the file's pose held by PD targets at its own hinge angles (gain KP,
// uncapped), ground on; one environment stepped STEPS times, then a Batch of
// ENVS copies stepped STEPS times, after two untimed steps each.
static int throughput(const char *model, int envs, int steps, double dt, int iterations,
                      double kp) {
  Solver sim;
  sim.load(model);
  sim.options.dt = dt;
  sim.options.iterations = iterations;
  sim.options.ground = true;
  for (auto &j : sim.joints) {
    j.kp = kp;
    j.target = sim.angle(j);
  }
  using clock = std::chrono::steady_clock;
  auto seconds = [](clock::time_point a, clock::time_point b) {
    return std::chrono::duration<double>(b - a).count();
  };
  Solver one = sim;
  one.step();
  one.step();
  auto t0 = clock::now();
  for (int s = 0; s < steps; ++s)
    one.step();
  const double single = seconds(t0, clock::now());
  Batch batch(sim, envs);
  batch.step();
  batch.step();
  t0 = clock::now();
  for (int s = 0; s < steps; ++s)
    batch.step();
  const double many = seconds(t0, clock::now());
  int failed = 0;
  for (const Solver &e : batch.environments)
    failed += std::isfinite(e.bodies.at(1).x.z) ? 0 : 1;
  std::printf("single env: %.1f steps/s (%.3f ms per step)\n", steps / single,
              1e3 * single / steps);
  std::printf("batch of %d: %.1f env-steps/s (%.3f ms per Batch::step), %d non-finite\n", envs,
              double(envs) * steps / many, 1e3 * many / steps, failed);
  return failed ? 1 : 0;
}

// One environment stepped STEPS times with Solver::stepImplicit (dt 5 ms, 10
// iterations, the file's controls); prints "step body x y z qw qx qy qz" for
// every body after every step, full precision.
static int trace(const char *model, int steps) {
  Solver sim;
  sim.load(model);
  sim.options.dt = 0.005;
  sim.options.iterations = 10;
  for (int s = 1; s <= steps; ++s) {
    sim.stepImplicit();
    for (size_t b = 0; b < sim.bodies.size(); ++b) {
      const Body &x = sim.bodies[b];
      std::printf("%d %zu %.17g %.17g %.17g %.17g %.17g %.17g %.17g\n", s, b, x.x.x, x.x.y,
                  x.x.z, x.q.w, x.q.x, x.q.y, x.q.z);
    }
  }
  return 0;
}

int main(int argc, char **argv) {
  try {
    if (argc >= 2 && std::strcmp(argv[1], "math") == 0)
      return math();
    if (argc >= 3 && std::strcmp(argv[1], "gpu") == 0)
      return gpu(argv[2]);
    if (argc >= 4 && std::strcmp(argv[1], "trace") == 0)
      return trace(argv[2], std::atoi(argv[3]));
    if (argc >= 3 && std::strcmp(argv[1], "batch") == 0)
      return batch(argv[2]);
    if (argc >= 6 && std::strcmp(argv[1], "seqtrace") == 0)
      return seqtrace(argv[2], std::atoi(argv[3]), std::atof(argv[4]), std::atoi(argv[5]),
                      argc >= 7 ? argv[6] : nullptr);
    if (argc >= 8 && std::strcmp(argv[1], "throughput") == 0)
      return throughput(argv[2], std::atoi(argv[3]), std::atoi(argv[4]), std::atof(argv[5]),
                        std::atoi(argv[6]), std::atof(argv[7]));
    std::fprintf(stderr, "usage: solver_api_test math | gpu MODEL | batch MODEL | trace MODEL "
                         "STEPS | seqtrace MODEL STEPS DT ITER [CONTROLS] | throughput MODEL "
                         "ENVS STEPS DT ITER KP\n");
    return 2;
  } catch (const std::exception &e) {
    std::fprintf(stderr, "FAILED: %s\n", e.what());
    return 1;
  }
}
