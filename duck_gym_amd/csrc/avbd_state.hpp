// Data layout of the batched AVBD step on gfx950.
//
// HBM: one contiguous `EnvState` blob per environment (env-major), holding
// exactly the state that survives between launches: body poses/velocities,
// per-env mass and inertia, joint multipliers and penalties, the last
// controls, the compacted ground and self contact lists (warm-start cache),
// diagnostics and the failure flag.  A workgroup copies its environments'
// blobs into LDS once per launch (live contacts only) and back at the end.
//
// LDS: `EnvLds` = `EnvState` + per-step scratch (x0/q0/xp/qp, joint c0 and
// angle0, colour schedule, per-body contact masks), one per environment of
// the workgroup, plus one `Frames` copy of the shared joint model.
//
// Fields are structure-of-arrays indexed [component][body|joint] so that the
// lanes of one environment, which work on different bodies or joints, touch
// consecutive LDS words.
#pragma once
#include "avbd_math.hpp"

#include <cstdint>

namespace duckhip {

constexpr int kMaxModelBodies = 32, kMaxModelJoints = 32, kMaxModelShapes = 32,
              kMaxModelPairs = 32;
// Point-set shapes with at most this many points are staged in LDS and keep
// their candidate heights in registers during ground-contact selection.
constexpr int kCachedPoints = 8;

// Read-only model in global memory (one copy per batch).
template <class R> struct DeviceModel {
  int nb, nj, ns, np, ground, iterations, groundCapacity, selfCapacity;
  R dt, tolerance, alpha, gamma, betaLinear, betaAngular;
  R gravity[3];
  // bodies in the file state
  R mass[kMaxModelBodies], inertia[3][kMaxModelBodies], x[3][kMaxModelBodies],
      q[4][kMaxModelBodies], v[3][kMaxModelBodies], w[3][kMaxModelBodies];
  int colors[kMaxModelBodies];
  // joints: frames (as in Frames) and file values of the per-env parameters
  int ja[kMaxModelJoints], jb[kMaxModelJoints], limited[kMaxModelJoints];
  R ra[3][kMaxModelJoints], rb[3][kMaxModelJoints], axisA[3][kMaxModelJoints],
      axisB[3][kMaxModelJoints], tangentA[3][kMaxModelJoints], tangentB[3][kMaxModelJoints];
  R lo[kMaxModelJoints], hi[kMaxModelJoints], armature[kMaxModelJoints];
  int adjStart[kMaxModelBodies + 1], adj[2 * kMaxModelJoints];
  // adjacency entries packed as hinge | body a << 8 | body b << 16, and the
  // default colour schedule (dynamic bodies of colour 0 then 1, index order)
  int adjPacked[2 * kMaxModelJoints], order[kMaxModelBodies], colorStart[3];
  R damping[kMaxModelJoints], frictionloss[kMaxModelJoints], torque[kMaxModelJoints],
      kp[kMaxModelJoints], target[kMaxModelJoints], maxTorque[kMaxModelJoints],
      originalAngle[kMaxModelJoints];
  // shapes
  int sbody[kMaxModelShapes], stype[kMaxModelShapes], sground[kMaxModelShapes],
      soffset[kMaxModelShapes], scount[kMaxModelShapes];
  R center[3][kMaxModelShapes], size[3][kMaxModelShapes], sq[4][kMaxModelShapes],
      sfriction[kMaxModelShapes], radius[kMaxModelShapes], interior[3][kMaxModelShapes];
  // ground detection: bit 0 ground contact enabled (model and shape), bit 1
  // point set of at most kCachedPoints points, whose points are spts
  int sflags[kMaxModelShapes];
  R spts[kCachedPoints][3][kMaxModelShapes];
  // body-contact pairs (shape indices)
  int pa[kMaxModelPairs], pb[kMaxModelPairs];
  R pfriction[kMaxModelPairs];
  // tree levels of the Newton-Euler load pass: a hinge's level is the depth
  // of its child body (a body that is no hinge's child has depth 0);
  // jointLevels = the deepest level, or 0 when the hinges do not form a tree
  // listed parent first (the pass then runs in hinge order on one lane)
  int jointLevel[kMaxModelJoints], bodyLevel[kMaxModelBodies], jointLevels;
  unsigned childHinges[kMaxModelBodies]; // bit j: hinge j has this body as parent
};

// Joint model used inside the solve, staged in LDS once per workgroup.
template <class R, int B, int J> struct alignas(16) Frames {
  int a[J], b[J], limited[J];
  R ra[3][J], rb[3][J], axisA[3][J], axisB[3][J], tangentA[3][J], tangentB[3][J];
  R lo[J], hi[J], armature[J];
  int adjStart[B + 1];
  int adj[2 * J]; // hinge | body a << 8 | body b << 16, grouped by body
  R shapeFriction[kMaxModelShapes];
  // Colour schedule without body-body contacts (model colours, bodies of
  // non-zero model mass in index order within each colour).
  int order[B], colorStart[3];
  // Detection data per shape (shapes <= B) and model masses.  sflags: the
  // model's bits (1 ground contact, 2 staged point set) | shape type << 4.
  // spt holds the points of a staged point set; a sphere or capsule has no
  // points and holds its centre (spt[0]), radius and half length (spt[1]
  // [0..1]) and capsule axis (spt[2]) there instead.
  int sbody[B], sflags[B], scount[B];
  R sradius[B], mass[B];
  R spt[kCachedPoints][3][B];
  R sinterior[3][B];
  int pair[B]; // body-contact pairs: shape a | shape b << 8 (pairs <= B)
};

// Ground contact (normal = +z, anchor on the plane).  id packs
// shape (bits 0-5), body (6-11), feature (12-30) and stick (31).
template <class R> struct GroundContact {
  int id;
  R local[3], anchor[2], c0, lambda[3], penalty[3];
};
// Body-body contact.  id packs body (0-5), other (6-11), shape (12-17),
// otherShape (18-23), stick (31).
template <class R> struct SelfContact {
  int id;
  R local[3], localB[3], t1[3], t2[3], n[3], c0, friction, lambda[3], penalty[3];
};

// In the double layout the four bytes after `id` are alignment padding:
// kept at zero in every contact written, so that a state blob holds no
// indeterminate bytes (checkpoints compare and replay bit for bit).
template <class C> DUCK_HD void clearContactPadding(C &c) {
  if constexpr (offsetof(C, local) == 2 * sizeof(int))
    reinterpret_cast<int *>(&c)[1] = 0;
}

DUCK_HD int gcShape(int id) { return id & 63; }
DUCK_HD int gcBody(int id) { return (id >> 6) & 63; }
DUCK_HD int gcFeature(int id) { return (id >> 12) & 0x7ffff; }
DUCK_HD bool gcStick(int id) { return id < 0; }
// the shape and feature fields of a ground-contact id
constexpr int kGcShapeFeature = 63 | (0x7ffff << 12);
DUCK_HD int gcPack(int shape, int body, int feature, bool stick) {
  return shape | (body << 6) | (feature << 12) | (stick ? int(0x80000000u) : 0);
}
DUCK_HD int scBody(int id) { return id & 63; }
DUCK_HD int scOther(int id) { return (id >> 6) & 63; }
DUCK_HD int scShape(int id) { return (id >> 12) & 63; }
DUCK_HD int scOtherShape(int id) { return (id >> 18) & 63; }
DUCK_HD bool scStick(int id) { return id < 0; }
DUCK_HD int scPack(int body, int other, int shape, int otherShape, bool stick) {
  return body | (other << 6) | (shape << 12) | (otherShape << 18) |
         (stick ? int(0x80000000u) : 0);
}

enum DiagSlot { kJointError, kPenetration, kContacts, kConverged, kAxisError, kIterations };

// Persistent per-env state; the HBM blob is exactly this struct.  Its fields
// are grouped by what a step does with them:
//  0. the step diagnostics, and the last controls' targets and external
//     force: written by every launch that steps the environment or sets them,
//     read only by one that holds its controls or sets motor channels (which
//     keep the targets; a step starts the diagnostics afresh); they end where
//     group 1 starts, so a launch writes them and group 1 as one range;
//  1. read and written by every step, from a 128-byte boundary of the blob
//     through the live entries of the ground-contact list (one contiguous
//     range), then the live body contacts;
//  2. the drive parameters of the last controls (kp through damping): read
//     only by a launch that holds its controls, written only when they
//     change.  `drive` records what they hold: kDriveTarget -- kp and
//     maxTorque are `driveKp`/`driveLimit` and torque, frictionloss and
//     damping the model's, on every hinge (zeros past the last); kDriveMotor
//     -- kp and maxTorque are zero; kDriveOther -- no claim.  A target launch
//     with the same kp and limit, and a motor launch after a motor launch,
//     find their values in place and skip the rewrite;
//  3. the colouring of the last step: written only when it differs from what
//     the blob holds; `modelColours` records that the blob holds the model's
//     colours (zeros past the last body);
//  4. set by reset only; a launch reads them only when some environment's
//     may differ from the model's (reset with per-env extensions, imported
//     states), and never writes them back.
// Every claim of `drive` and `modelColours` holds for the blob's bytes: the
// writers keep them so, and an import clears any that the imported bytes do
// not bear out.  `lead` (never copied, zero as created) places group 1 on the
// 128-byte boundary.
enum DriveKind { kDriveOther = 0, kDriveTarget = 1, kDriveMotor = 2 };
template <class R, int J> constexpr int leadBytes() {
  constexpr int controls = int(sizeof(R)) * (8 + J + 3);
  return (controls + 4 + 127) / 128 * 128 - controls;
}
template <class R, int B, int J, int CG, int CS> struct EnvState {
  unsigned char lead[leadBytes<R, J>()];
  R diag[8];
  R target[J];
  R force[3];
  R x[3][B];
  R q[4][B], v[3][B], w[3][B];
  R lambda[7][J], penalty[7][J];
  R lambdaF[J], penaltyF[J];
  int failed, ngc, nsc, colorCount;
  int drive, modelColours;
  R driveKp, driveLimit;
  alignas(16) GroundContact<R> gc[CG];
  SelfContact<R> sc[CS];
  alignas(16) R kp[J];
  R maxTorque[J], torque[J], frictionloss[J], damping[J];
  alignas(16) int colors[B]; // model colours + fresh ones
  alignas(16) R mass[B], inertia[3][B];
  R friction; // per-env ground friction; < 0 selects the shape friction
};

template <class R, int B, int J, int CG, int CS> struct EnvLdsCore {
  EnvState<R, B, J, CG, CS> s;
  // per-step scratch
  R x0[3][B], q0[4][B], xp[3][B], qp[4][B];
  R Iw[6][B]; // world inertia at q0 (xx yy zz xy xz yz)
  R c0[7][J], angle0[J], velocity0[J];
  R stepDiag[8];
  // per body: bit i of word i / 64 = ground contact i belongs to the body;
  // bit i = body-body contact i involves it
  uint64_t gmask[(CG + 63) / 64][B];
  uint32_t smask[B];
  int order[B], colorStart[CS + 3];
  // what the write-back copies, decided with the controls: the first word
  // (bits 8-), the drive parameters (bits 1-2), and whether the blob held the
  // model's colours (bit 0); whether this step's third colour is assembled a
  // pass ahead of its solve, and then its body's body-contact mask (its
  // smask word is zero while the other rows are assembled)
  int writeback, early;
  uint32_t earlyMask;
  int pad2;
  int shapeCount[B]; // shapes <= B
  int pairHit[CS];   // body-contact pairs <= CS
  // a two-part body system assembled a pass ahead of its solve (21 Hessian
  // entries and 6 gradient entries per part; float batches only)
  R staged[sizeof(R) == sizeof(float) ? 2 : 1][28];
};

// One environment's LDS record.  A wave holds 64 / L environments and their
// lanes read the same field at consecutive words, so the record stride is
// padded to an odd multiple of L words: the environments of a wave then fall
// on disjoint LDS banks (32 or 64 banks of 4 bytes).
template <int Words, int L> constexpr int bankPadWords() { return (L - Words % (2 * L) + 2 * L) % (2 * L); }
template <class R, int B, int J, int CG, int CS, int L,
          int Pad = bankPadWords<int(sizeof(EnvLdsCore<R, B, J, CG, CS>) / 4), L>()>
struct EnvLds : EnvLdsCore<R, B, J, CG, CS> {
  int bankPad[Pad];
};
template <class R, int B, int J, int CG, int CS, int L>
struct EnvLds<R, B, J, CG, CS, L, 0> : EnvLdsCore<R, B, J, CG, CS> {};

// Byte offsets of the ground-contact list inside the blob (only its live
// entries are copied), of the diagnostics, the targets, the force and group 1,
// and the byte
// ranges of the drive parameters, of the
// three motor-written ones (torque through damping), of the colouring and of
// the reset-only group.
template <class S> constexpr size_t headerBytes() { return offsetof(S, gc); }
template <class S> constexpr size_t diagBegin() { return offsetof(S, diag); }
template <class S> constexpr size_t targetBegin() { return offsetof(S, target); }
template <class S> constexpr size_t forceBegin() { return offsetof(S, force); }
template <class S> constexpr size_t hotBegin() { return offsetof(S, x); }
template <class S> constexpr size_t driveBegin() { return offsetof(S, kp); }
template <class S> constexpr size_t motorBegin() { return offsetof(S, torque); }
template <class S> constexpr size_t driveEnd() { return offsetof(S, damping) + sizeof(S::damping); }
template <class S> constexpr size_t coloursBegin() { return offsetof(S, colors); }
template <class S> constexpr size_t coloursEnd() { return offsetof(S, colors) + sizeof(S::colors); }
template <class S> constexpr size_t resetBegin() { return offsetof(S, mass); }

} // namespace duckhip
