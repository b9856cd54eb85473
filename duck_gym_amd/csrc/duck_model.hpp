// Host side of the drop-in boundary: `.duck` text model -> flat model tables.
//
// Parses the v1/v2 text format with the validation of src/solver.cpp:67-174
// and flattens it with the checks of src/cuda/model.hpp:20-143 (capacity,
// single-parent tree in topological order, depth-parity colours, bipartite
// hinge graph, body->joint CSR, shape points and interior points).
#pragma once
#include <istream>
#include <string>
#include <vector>

namespace duckhip {

struct HostBody {
  std::string name;
  double mass = 0, inertia[3]{}, x[3]{}, q[4]{1, 0, 0, 0}, v[3]{}, w[3]{};
};
struct HostJoint {
  std::string name;
  int a = 0, b = 0;
  double ra[3]{}, rb[3]{}, axisA[3]{}, axisB[3]{}, tangentA[3]{}, tangentB[3]{};
  int limited = 0;
  double lo = 0, hi = 0, damping = 0, armature = 0, frictionloss = 0, torque = 0, kp = 0,
         target = 0, maxTorque = 0;
};
struct HostShape {
  int body = 0, type = 0, ground = 1, offset = 0, count = 0;
  double center[3]{}, size[3]{}, q[4]{1, 0, 0, 0}, friction = 0.8, radius = 0, interior[3]{};
  std::vector<double> vertices; // the file's hull vertices (xyz), shape frame
};
struct HostPair {
  int a = 0, b = 0;
  double friction = 0;
};

struct HostModel {
  double gravity[3]{0, 0, -9.81};
  int ground = 0;
  std::vector<HostBody> bodies;
  std::vector<HostJoint> joints;
  std::vector<HostShape> shapes;
  std::vector<HostPair> pairs;
  std::vector<double> points; // xyz triples, body frame, shape offsets index this
  std::vector<int> colors, adjacencyStart, adjacency;
  int groundCapacity = 0, selfCapacity = 0;
};

// Throws std::invalid_argument / std::runtime_error with the reference's
// messages on malformed input.
HostModel loadModel(const std::string &path);
// The two halves of loadModel: parse the text with the checks of
// Solver::load (std::runtime_error), and flatten it with the checks of
// convert (std::invalid_argument): capacities, tree order, colours,
// adjacency, shape points, interiors and contact capacities.
HostModel parseModel(const std::string &path);
void flattenModel(HostModel &m);
// loadModel on the text of a `.duck` file held in memory (the same checks
// and messages); parseModelStream is parseModel on an open stream.
HostModel loadModelText(const std::string &text);
HostModel parseModelStream(std::istream &in);

} // namespace duckhip
