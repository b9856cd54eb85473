// Host code under AddressSanitizer and UndefinedBehaviorSanitizer (the role
// of the reference's DUCK_SANITIZE build, CMakeLists.txt:6-14): the product's
// `.duck` loader (duck_gym_amd/csrc/duck_model.cpp) and the CPU oracle
// (oracle/avbd_oracle.cpp), linked into one program built with
// -fsanitize=address,undefined.
//
//   sanitize_driver load FILE...   parse and flatten each file; prints
//                                  "ok" or the error message per file
//   sanitize_driver step FILE...   each model in both oracle modes (the
//                                  explicit-sequential one rejects body
//                                  pairs) and both precisions: reset, 30
//                                  steps under seeded controls, every query
// Exits non-zero when a sanitizer reports (halt_on_error) or a step fails.
#include "../../duck_gym_amd/csrc/duck_model.hpp"
#include "../../oracle/avbd_oracle.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

static int load(int n, char **files) {
  for (int i = 0; i < n; ++i) {
    try {
      duckhip::HostModel m = duckhip::loadModel(files[i]);
      std::printf("ok %s %zu %zu %zu\n", files[i], m.bodies.size(), m.joints.size(),
                  m.shapes.size());
    } catch (const std::exception &e) {
      std::printf("error %s: %s\n", files[i], e.what());
    }
  }
  return 0;
}

static int step(int n, char **files) {
  std::mt19937_64 rng(20260927);
  std::uniform_real_distribution<double> u(-0.3, 0.3);
  for (int i = 0; i < n; ++i)
    for (int mode = 0; mode < 2; ++mode)
      for (int fp64 = 0; fp64 < 2; ++fp64) {
        void *h = oracle_create(files[i], 0.005, 10, fp64, mode);
        if (!h) {
          // the explicit-sequential mode has no body-body contact (solver.cpp)
          std::printf("rejected %s mode %d: %s\n", files[i], mode, oracle_last_error());
          if (mode == 0)
            return 1;
          continue;
        }
        int nb = 0, nj = 0;
        oracle_dims(h, &nb, &nj);
        std::vector<double> q(nj), root(6, 0), target(nj), force(3, 0);
        for (auto &v : q)
          v = u(rng);
        oracle_reset(h, q.data(), root.data());
        std::vector<double> bodies(13 * nb), joints(2 * nj), diag(6), js(31 * nj),
            forces(3 * nb), stats(2), counts(2), loads(3 * nj), reals(26 * 256), motor(3 * nj);
        std::vector<int> ints(6 * 256), colors(nb);
        for (int s = 0; s < 30; ++s) {
          for (auto &v : target)
            v = u(rng);
          force[0] = u(rng);
          if (s % 3 == 2) {
            for (int j = 0; j < nj; ++j) {
              motor[3 * j] = u(rng);
              motor[3 * j + 1] = std::abs(u(rng)) * 0.1;
              motor[3 * j + 2] = std::abs(u(rng));
            }
            oracle_set_motor(h, motor.data(), force.data());
          } else {
            oracle_set_controls(h, target.data(), force.data(), 8.0, s % 2 ? 0.0 : 0.5);
          }
          if (oracle_advance(h, 1))
            std::printf("step error %s: %s\n", files[i], oracle_last_error());
          oracle_snapshot(h, bodies.data(), joints.data(), diag.data());
          int count = 0, colorCount = 0;
          oracle_contacts(h, 256, &count, ints.data(), reals.data());
          oracle_colors(h, colors.data(), &colorCount);
          oracle_joint_state(h, js.data());
          oracle_contact_forces(h, s % 2, forces.data());
          oracle_self_contact_stats(h, stats.data());
          oracle_contact_counts(h, counts.data());
          oracle_generalized_loads(h, root.data(), loads.data());
        }
        std::printf("stepped %s mode %d fp64 %d failed %d\n", files[i], mode, fp64,
                    oracle_failed(h));
        oracle_destroy(h);
      }
  // the threaded batch: 5 environments on 3 workers, one reset with a
  // non-finite pose, target and motor steps, every query
  for (int i = 0; i < n; ++i)
    for (int fp64 = 0; fp64 < 2; ++fp64) {
      void *b = oracle_batch_create(files[i], 5, 0.005, 10, fp64, 3);
      if (!b) {
        std::printf("batch rejected %s: %s\n", files[i], oracle_last_error());
        return 1;
      }
      int ne = 0, nb = 0, nj = 0;
      oracle_batch_dims(b, &ne, &nb, &nj);
      std::vector<unsigned char> mask(ne, 1);
      std::vector<double> q(ne * nj), root(ne * 6, 0), target(ne * nj), forces(ne * 3, 0),
          motor(ne * nj * 3), bodies(ne * nb * 13), joints(ne * nj * 2), diag(ne * 6),
          counts(ne * 2);
      for (auto &v : q)
        v = u(rng);
      root[6 * 2] = NAN;
      oracle_batch_reset(b, mask.data(), q.data(), root.data());
      for (int s = 0; s < 6; ++s) {
        for (auto &v : target)
          v = u(rng);
        if (s == 3) {
          for (int k = 0; k < ne * nj; ++k) {
            motor[3 * k] = u(rng);
            motor[3 * k + 1] = std::abs(u(rng)) * 0.1;
            motor[3 * k + 2] = std::abs(u(rng));
          }
          oracle_batch_step_motor(b, motor.data(), forces.data());
        } else if (oracle_batch_step(b, target.data(), forces.data(), 1, 8.0, 1e9)) {
          std::printf("batch step error %s: %s\n", files[i], oracle_last_error());
          return 1;
        }
        oracle_batch_state(b, bodies.data(), joints.data(), diag.data());
        oracle_batch_contact_counts(b, counts.data());
      }
      std::printf("batch stepped %s fp64 %d\n", files[i], fp64);
      oracle_batch_destroy(b);
    }
  // the stand-alone narrow phase: two boxes' corners, overlapping
  std::vector<double> box;
  for (int c = 0; c < 8; ++c)
    for (int k = 0; k < 3; ++k)
      box.push_back(((c >> k) & 1) ? 0.05 : -0.05);
  const double poses[14] = {0, 0, 0, 1, 0, 0, 0, 0.08, 0.01, 0.0, 1, 0, 0, 0};
  double out[8];
  for (int fp64 = 0; fp64 < 2; ++fp64)
    if (oracle_convex_query(box.data(), 8, box.data(), 8, poses, 0.0, 1e-8, fp64, out) ||
        out[0] != 1) {
      std::printf("convex query failed\n");
      return 1;
    }
  std::printf("convex query ok depth %.6f\n", out[1]);
  return 0;
}

int main(int argc, char **argv) {
  if (argc >= 3 && std::strcmp(argv[1], "load") == 0)
    return load(argc - 2, argv + 2);
  if (argc >= 3 && std::strcmp(argv[1], "step") == 0)
    return step(argc - 2, argv + 2);
  std::fprintf(stderr, "usage: sanitize_driver load|step FILE...\n");
  return 2;
}
