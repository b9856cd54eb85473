// The duck C++ solver interface (include/duck/solver.hpp of duck_gym: the
// same types, fields, defaults and methods), stepped on the GPU.
//
// A Solver holds one environment's model and state in its public members, as
// the reference's does; callers may read and change them between steps.
// step() is the reference's Solver::step (src/solver.cpp:315-537): the PD
// drive as an explicit torque in the predictor, block Gauss-Seidel over the
// bodies in index order, ground contacts, the warm-start fields angle0 /
// velocity0 / c0 kept on the hinges and every Diagnostics field.  It runs on
// the MI355X through duck_sequential_step (libduck_hip.so, one GPU thread per
// environment, float64): the public state goes to the device, is stepped and
// comes back, and the same errors are thrown as std::runtime_error ("Body
// contacts require the shared CpuBatch/CUDA solver", "Invalid solver
// options", "Non-positive local Hessian", "Non-finite state", "Zero
// quaternion").  Batch::step steps all its environments in one launch.
//
// stepImplicit() is the reference's CUDA batch step instead (src/cuda/
// kernel.cuh: the PD drive stamped implicitly into each body's Hessian,
// graph-coloured block descent, body-body contacts), which stays stable where
// the explicit drive diverges (the MicroDuck biped at kp = 8 and dt = 5 ms):
//  * Body::force is applied to the root body (body 1) only; it throws
//    std::invalid_argument for a non-zero force on any other body;
//  * Options::alpha, gamma, betaLinear, betaAngular and tolerance keep their
//    defaults (0.9, 0.99, 1e7, 1e5, 1e-7): it throws for other values;
//  * Diagnostics::update is not computed (0); Joint::angle0, velocity0 and
//    c0 are not written back; contacts are the ground contacts (body-body
//    contacts of two-way pairs are kept internally between steps).
// load() parses a `.duck` file with Solver::load's checks (solver.cpp:67-174,
// std::runtime_error); the first stepImplicit() also applies the batch's
// flattening checks (model.hpp: std::invalid_argument), e.g. at most 32 bodies.
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
  // One step with the reference's CUDA-batch semantics (see above).
  void stepImplicit();
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

// Solver::step of every environment in one GPU launch, with the outcome of
// stepping them one after the other: when an environment throws, those
// before it have stepped, it is left as its step left it, and those after it
// are untouched.
void stepAll(std::vector<Solver> &environments);

// Independent environments copied from a prototype; step() advances each.
class Batch {
public:
  std::vector<Solver> environments;
  Batch(const Solver &prototype, int num_envs) {
    if (num_envs < 1)
      throw std::invalid_argument("num_envs must be positive");
    environments.assign(num_envs, prototype);
  }
  void step() { stepAll(environments); }
  void reset(int id) { environments.at(id).reset(); }
};

} // namespace duck
