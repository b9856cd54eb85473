// Host side of the explicit-sequential step (duck_sequential_step): the
// checks an environment passes before its record reaches the device, the
// record layout the kernel walks (avbd_sequential.hpp) and the copies into
// and out of the callers' structs.  Host code only.
#pragma once
#include "../../include/duck_hip.h"
#include "avbd_sequential.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace duckhip {
namespace seq {

// An argument the step refuses (duck_sequential_step returns it as
// DUCK_ERR_ARGUMENT).
struct SeqError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
inline void check(bool ok, const char *message) {
  if (!ok)
    throw SeqError(message);
}

inline size_t alignUp(size_t n, size_t a) { return (n + a - 1) / a * a; }

// The checks an environment passes before its record reaches the device:
// the reference's option check (solver.cpp:318-320), every index the step
// dereferences in range, and the capacities the step writes into.
inline void checkSequential(const DuckSeqEnv &e, int steps) {
  const DuckSeqOptions &o = e.options;
  check(o.dt > 0 && o.iterations >= 1 && o.alpha >= 0 && o.alpha < 1 && o.gamma > 0 &&
            o.gamma < 1,
        "Invalid solver options");
  // a bound on one call's running time: a thread runs its environment's
  // iterations serially (about 0.1 ms each for a 15-body model)
  check(double(o.iterations) * steps <= 2e5,
        "sequential step: more than 2e5 iterations x steps in one call");
  check(e.num_bodies >= 0 && e.num_joints >= 0 && e.num_shapes >= 0 && e.num_points >= 0 &&
            e.num_contacts >= 0,
        "sequential step: negative count");
  check((e.bodies || !e.num_bodies) && (e.joints || !e.num_joints) &&
            (e.shapes || !e.num_shapes) && (e.points || !e.num_points) &&
            (e.contacts || !e.contact_capacity),
        "sequential step: null array");
  check(e.contact_capacity >= e.num_contacts && e.contact_capacity >= 4 * e.num_shapes,
        "sequential step: contact capacity below the contacts held or 4 per shape");
  for (int i = 0; i < e.num_joints; ++i) {
    const DuckSeqJoint &j = e.joints[i];
    check(j.a >= 0 && j.a < e.num_bodies && j.b >= 0 && j.b < e.num_bodies,
          "sequential step: hinge body index out of range");
  }
  for (int i = 0; i < e.num_shapes; ++i) {
    const DuckSeqShape &s = e.shapes[i];
    check(s.body >= 0 && s.body < e.num_bodies && s.type >= 0 && s.type <= 3,
          "sequential step: shape body or type out of range");
    check(s.type == 0 || s.type == 2 ||
              (s.first_point >= 0 && s.num_points >= 0 &&
               s.first_point + s.num_points <= e.num_points),
          "sequential step: shape points out of range");
  }
  for (int i = 0; i < e.num_contacts; ++i)
    check(e.contacts[i].body >= 0 && e.contacts[i].body < e.num_bodies,
          "sequential step: contact body index out of range");
}

// One environment's record: the header, then its arrays at 16-byte aligned
// offsets; the record's size is a multiple of 256 bytes.
inline SeqRecord layoutSequential(const DuckSeqEnv &e, size_t &bytes) {
  SeqRecord r{};
  r.options = e.options;
  r.bodies = e.num_bodies;
  r.joints = e.num_joints;
  r.shapes = e.num_shapes;
  r.points = e.num_points;
  r.contacts = e.num_contacts;
  r.candidates = 2;
  for (int i = 0; i < e.num_shapes; ++i)
    if (e.shapes[i].type == 1 || e.shapes[i].type == 3)
      r.candidates = std::max(r.candidates, e.shapes[i].num_points);
  size_t at = alignUp(sizeof(SeqRecord), 16);
  auto place = [&](long long &field, size_t size) {
    field = static_cast<long long>(at);
    at = alignUp(at + size, 16);
  };
  place(r.body, sizeof(DuckSeqBody) * e.num_bodies);
  place(r.joint, sizeof(DuckSeqJoint) * e.num_joints);
  place(r.shape, sizeof(DuckSeqShape) * e.num_shapes);
  place(r.point, sizeof(double) * 3 * e.num_points);
  // a step copies the last list into `old` and writes at most 4 contacts per
  // shape: both hold the input list and any later step's
  const int listCapacity = std::max(4 * e.num_shapes, e.num_contacts);
  place(r.contact, sizeof(DuckSeqContact) * listCapacity);
  place(r.old, sizeof(DuckSeqContact) * listCapacity);
  place(r.adjacencyStart, sizeof(int) * (e.num_bodies + 1));
  place(r.adjacency, sizeof(int) * 2 * e.num_joints);
  place(r.candidateZ, sizeof(double) * r.candidates);
  place(r.candidateK, sizeof(int) * r.candidates);
  place(r.torque, sizeof(double) * 3 * e.num_bodies);
  bytes = alignUp(at, 256);
  return r;
}

// The host image of every environment's record (offsets[i] = where record i
// starts), after checkSequential.
inline void packSequential(const DuckSeqEnv *envs, int n, std::vector<unsigned char> &image,
                    std::vector<long long> &offsets) {
  offsets.assign(n, 0);
  std::vector<SeqRecord> headers(n);
  size_t total = 0;
  for (int i = 0; i < n; ++i) {
    size_t bytes = 0;
    headers[i] = layoutSequential(envs[i], bytes);
    offsets[i] = static_cast<long long>(total);
    total += bytes;
  }
  image.assign(total, 0);
  for (int i = 0; i < n; ++i) {
    const DuckSeqEnv &e = envs[i];
    const SeqRecord &r = headers[i];
    unsigned char *base = image.data() + offsets[i];
    std::memcpy(base, &r, sizeof(r));
    auto put = [&](long long offset, const void *src, size_t size) {
      if (size)
        std::memcpy(base + offset, src, size);
    };
    put(r.body, e.bodies, sizeof(DuckSeqBody) * e.num_bodies);
    put(r.joint, e.joints, sizeof(DuckSeqJoint) * e.num_joints);
    put(r.shape, e.shapes, sizeof(DuckSeqShape) * e.num_shapes);
    put(r.point, e.points, sizeof(double) * 3 * e.num_points);
    put(r.contact, e.contacts, sizeof(DuckSeqContact) * e.num_contacts);
    // body -> hinge adjacency in hinge order (solver.cpp:103-104)
    std::vector<int> start(e.num_bodies + 1, 0), list(2 * e.num_joints);
    for (int j = 0; j < e.num_joints; ++j) {
      ++start[e.joints[j].a + 1];
      ++start[e.joints[j].b + 1];
    }
    for (int b = 0; b < e.num_bodies; ++b)
      start[b + 1] += start[b];
    std::vector<int> fill(start.begin(), start.end() - 1);
    for (int j = 0; j < e.num_joints; ++j) {
      list[fill[e.joints[j].a]++] = j;
      list[fill[e.joints[j].b]++] = j;
    }
    put(r.adjacencyStart, start.data(), sizeof(int) * start.size());
    put(r.adjacency, list.data(), sizeof(int) * list.size());
  }
}

// The stepped records back into the callers' structs.
inline void unpackSequential(DuckSeqEnv *envs, int n, const std::vector<unsigned char> &image,
                      const std::vector<long long> &offsets) {
  for (int i = 0; i < n; ++i) {
    DuckSeqEnv &e = envs[i];
    const unsigned char *base = image.data() + offsets[i];
    SeqRecord r;
    std::memcpy(&r, base, sizeof(r));
    auto get = [&](void *dst, long long offset, size_t size) {
      if (size)
        std::memcpy(dst, base + offset, size);
    };
    get(e.bodies, r.body, sizeof(DuckSeqBody) * e.num_bodies);
    get(e.joints, r.joint, sizeof(DuckSeqJoint) * e.num_joints);
    get(e.contacts, r.contact, sizeof(DuckSeqContact) * r.contacts);
    e.num_contacts = r.contacts;
    e.diagnostics = r.diagnostics;
    e.status = r.status;
  }
}

} // namespace seq
} // namespace duckhip
