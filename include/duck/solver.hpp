// The duck C++ solver interface (include/duck/solver.hpp of duck_gym: the
// same types, fields, defaults and methods), stepped on the GPU.
//
// A Solver holds one environment's model and state in its public members, as
// the reference's does; callers may read and change them between steps.
// step() runs one physics step of that state on the MI355X with the batched
// HIP step of libduck_hip.so (float64, one environment): the public state is
// written into a one-environment device batch, advanced once with the
// per-hinge controls it holds (target, kp, maxTorque, torque, frictionloss,
// damping) and the root body's force, and read back.  The step has the
// semantics of the reference's CUDA batch (src/cuda/kernel.cuh: the PD drive
// stamped implicitly into each body's Hessian, graph-coloured block descent,
// body-body contacts) rather than src/solver.cpp's explicit PD torque and
// body-order sweeps; on the MicroDuck biped at kp = 8 and dt = 5 ms the
// latter diverges.  Consequences for callers of the reference:
//  * Body::force is applied to the root body (body 1) only; step() throws
//    std::invalid_argument for a non-zero force on any other body;
//  * Options::alpha, gamma, betaLinear, betaAngular and tolerance keep their
//    defaults (0.9, 0.99, 1e7, 1e5, 1e-7): step() throws for other values;
//  * Diagnostics::update is not computed (0); Joint::angle0, velocity0 and
//    c0 are not written back; contacts are the ground contacts (body-body
//    contacts of two-way pairs are kept internally between steps).
// load() parses a `.duck` file with Solver::load's checks (solver.cpp:67-174,
// std::runtime_error); the first step() also applies the batch's flattening
// checks (model.hpp: std::invalid_argument), e.g. at most 32 bodies.
#pragma once
#include "math.hpp"

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace duck {

struct Body {
  std::string name;
  double mass = 0;
  Vec3 inertia{}, x{}, v{}, w{}, x0{}, xp{}, force{};
  Quat q{}, q0{}, qp{};
};
struct Joint {
  std::string name;
  int a = 0, b = 0;
  Vec3 ra{}, rb{}, axisA{}, axisB{}, tangentA{}, tangentB{};
  double lo = 0, hi = 0, damping = 0, armature = 0, frictionloss = 0, lambdaF = 0,
         penaltyF = 1, torque = 0, kp = 0, target = 0, maxTorque = 0;
  bool limited = false;
  double angle0 = 0, velocity0 = 0;
  std::array<double, 7> lambda{}, penalty{}, c0{};
};
struct Shape {
  int body = 0;
  Vec3 center{}, size{};
  Quat q{};
  int type = 0; // 0 sphere, 1 box, 2 capsule, 3 convex hull
  double friction = 0.8;
  std::vector<Vec3> vertices, localPoints;
  double boundingRadius = 0;
  bool ground = true;
};
struct CollisionPair {
  int a = 0, b = 0; // shape indices
  double friction = 0;
};
struct Contact {
  int body = 0, shape = 0, feature = 0;
  Vec3 local{}, anchor{};
  double radius = 0, friction = 0, c0 = 0;
  std::array<double, 3> lambda{}, penalty{};
  bool stick = false;
};
struct Options {
  double dt = 0.001, alpha = 0.9, gamma = 0.99, betaLinear = 1e7, betaAngular = 1e5,
         tolerance = 1e-7;
  int iterations = 100;
  Vec3 gravity{0, 0, -9.81};
  bool ground = false;
};
struct Diagnostics {
  double jointError = 0, axisError = 0, penetration = 0, update = 0;
  int contacts = 0, iterations = 0;
  bool converged = false;
};

class Solver {
public:
  Options options;
  std::vector<Body> bodies;
  std::vector<Joint> joints;
  std::vector<Shape> shapes;
  std::vector<CollisionPair> collisionPairs;
  std::vector<Contact> contacts;
  Diagnostics diagnostics;

  Solver();
  Solver(const Solver &other);
  Solver &operator=(const Solver &other);
  ~Solver();

  void load(const std::string &path);
  void step();
  void reset();
  // Hinge angle of b relative to a about the axis (solver.cpp:181-187).
  double angle(const Joint &j) const;
  // The seven constraint rows of a hinge and their Jacobians on both bodies:
  // anchor x, y, z; the two axis alignments; lower and upper limit.
  void evaluateJoint(const Joint &j, std::array<double, 7> &C, std::array<V6, 7> &JA,
                     std::array<V6, 7> &JB) const;

private:
  std::vector<Body> initialBodies;
  std::vector<Joint> initialJoints;
  struct Device;                  // the one-environment device batch
  std::unique_ptr<Device> device; // never shared: a copy makes its own
  std::vector<unsigned char> bodyContacts; // body-body contacts between steps
};

// Independent environments copied from a prototype; step() advances each.
class Batch {
public:
  std::vector<Solver> environments;
  Batch(const Solver &prototype, int num_envs) {
    if (num_envs < 1)
      throw std::invalid_argument("num_envs must be positive");
    environments.assign(num_envs, prototype);
  }
  void step() {
    for (auto &env : environments)
      env.step();
  }
  void reset(int id) { environments.at(id).reset(); }
};

} // namespace duck
