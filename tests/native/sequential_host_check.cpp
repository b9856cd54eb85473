// The explicit-sequential step's own code (duck_gym_amd/csrc/
// avbd_sequential.hpp, the body of sequentialStepKernel) compiled for the
// host and driven through the library's record packing
// (avbd_sequential_pack.hpp) and duck::Solver's conversions
// (duck_solver.cpp): with the host's libm it must reproduce the reference's
// duck_sim bit for bit, which separates the algorithm from the device's
// transcendental functions.  Test infrastructure: the library itself steps
// only on the GPU.
//
//   sequential_host_check MODEL STEPS DT ITER [CONTROLS]
//
// prints what `solver_api_test seqtrace` prints: per step one line per body,
// "s b x y z qw qx qy qz vx vy vz wx wy wz", then
// "d s jointError axisError penetration update contacts iterations converged".
#include "../../duck_gym_amd/csrc/duck_solver.cpp"
#include "avbd_sequential_pack.hpp"

#include <fstream>

int main(int argc, char **argv) {
  if (argc < 5) {
    std::fprintf(stderr, "usage: sequential_host_check MODEL STEPS DT ITER [CONTROLS]\n");
    return 2;
  }
  try {
    duck::Solver s;
    s.load(argv[1]);
    const int steps = std::atoi(argv[2]);
    s.options.dt = std::atof(argv[3]);
    s.options.iterations = std::atoi(argv[4]);
    if (argc > 5) {
      std::ifstream in(argv[5]);
      for (auto &j : s.joints)
        in >> j.target;
      double kp = 0, limit = 0;
      in >> kp >> limit >> s.bodies.at(1).force.x >> s.bodies[1].force.y >> s.bodies[1].force.z;
      if (!in)
        throw std::runtime_error("truncated controls file");
      for (auto &j : s.joints) {
        j.kp = kp;
        j.maxTorque = limit;
      }
    }
    for (int k = 1; k <= steps; ++k) {
      duck::SequentialStage st;
      duck::stage(s, st);
      DuckSeqEnv env = st.env;
      duckhip::seq::checkSequential(env, 1);
      std::vector<unsigned char> image;
      std::vector<long long> offsets;
      duckhip::seq::packSequential(&env, 1, image, offsets);
      duckhip::seq::Env(image.data() + offsets[0]).step();
      duckhip::seq::unpackSequential(&env, 1, image, offsets);
      st.env = env;
      duck::unstage(st, s);
      if (env.status) {
        std::fprintf(stderr, "fault %d at step %d\n", env.status, k);
        return 1;
      }
      for (size_t b = 0; b < s.bodies.size(); ++b) {
        const duck::Body &x = s.bodies[b];
        std::printf("%d %zu %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g %.17g "
                    "%.17g %.17g\n",
                    k, b, x.x.x, x.x.y, x.x.z, x.q.w, x.q.x, x.q.y, x.q.z, x.v.x, x.v.y, x.v.z,
                    x.w.x, x.w.y, x.w.z);
      }
      const duck::Diagnostics &d = s.diagnostics;
      std::printf("d %d %.17g %.17g %.17g %.17g %d %d %d\n", k, d.jointError, d.axisError,
                  d.penetration, d.update, d.contacts, d.iterations, d.converged ? 1 : 0);
    }
  } catch (const std::exception &e) {
    std::fprintf(stderr, "FAILED: %s\n", e.what());
    return 1;
  }
  return 0;
}
