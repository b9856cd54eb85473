// C ABI of the gfx950 AVBD batch (include/duck_hip.h): model upload, state
// ownership, stream ordering and kernel dispatch.
#include "../../include/duck_hip.h"
#include "avbd_sequential.hpp"
#include "avbd_sequential_pack.hpp"
#include "avbd_servo.hpp"
#include "avbd_task.hpp"
#include "duck_model.hpp"

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

// Device scratch of duck_reference_noalloc: one environment's state blob
// followed by its inputs and outputs.  Every device that runs this library
// holds its own copy for the life of the process; host code uses the address
// hipGetSymbolAddress returns for the current device (referenceScratch), never
// this name, which on the host is a stand-in and no device address.
constexpr size_t kReferenceScratchBytes = 64 * 1024;
static __device__ __align__(256) unsigned char scratch[kReferenceScratchBytes];

namespace duckhip {
namespace {

thread_local std::string g_lastError;

struct DuckError : std::runtime_error {
  int code;
  DuckError(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void hipCheck(hipError_t err, const char *what) {
  if (err != hipSuccess)
    throw DuckError(DUCK_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(err));
}
void require(bool ok, const std::string &message) {
  if (!ok)
    throw DuckError(DUCK_ERR_ARGUMENT, message);
}

// The device address of `scratch` on the current device `device`, looked up
// once per device (at the first batch created there) and kept.
void *referenceScratch(int device) {
  static std::mutex guard;
  static std::vector<void *> address;
  std::lock_guard<std::mutex> lock(guard);
  if (device >= int(address.size()))
    address.resize(device + 1, nullptr);
  if (!address[device]) {
    void *p = nullptr;
    hipCheck(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    address[device] = p;
  }
  return address[device];
}

// The host lock of a device's `scratch`: duck_reference_noalloc holds it for
// the whole call, so calls from several host threads on one device take turns
// instead of overwriting each other's blob and outputs.  A plain static
// mutex per device (no device memory).
constexpr int kMaxScratchDevices = 64;
std::mutex &referenceScratchLock(int device) {
  static std::mutex locks[kMaxScratchDevices];
  if (device < 0 || device >= kMaxScratchDevices)
    throw DuckError(DUCK_ERR_ARGUMENT, "reference scratch: device index " +
                                           std::to_string(device) + " beyond the library's " +
                                           std::to_string(kMaxScratchDevices));
  return locks[device];
}

// Clears `words` 32-bit words (a fill kernel rather than hipMemset, so that
// the sequence stays capturable).
__global__ void zeroWordsKernel(unsigned *p, long long words) {
  for (long long i = blockIdx.x * 64ll + threadIdx.x; i < words; i += 64ll * gridDim.x)
    p[i] = 0;
}

// Makes `device` current for the lifetime of the guard.
struct DeviceGuard {
  int previous = -1;
  explicit DeviceGuard(int device) {
    hipCheck(hipGetDevice(&previous), "hipGetDevice");
    if (previous != device)
      hipCheck(hipSetDevice(device), "hipSetDevice");
  }
  ~DeviceGuard() {
    int now = -1;
    if (hipGetDevice(&now) == hipSuccess && now != previous && previous >= 0)
      (void)hipSetDevice(previous);
  }
};

template <class R> DeviceModel<R> pack(const HostModel &h, double dt, int iterations) {
  DeviceModel<R> m;
  std::memset(&m, 0, sizeof(m));
  m.nb = h.bodies.size();
  m.nj = h.joints.size();
  m.ns = h.shapes.size();
  m.np = h.pairs.size();
  m.ground = h.ground;
  m.iterations = iterations;
  m.groundCapacity = h.groundCapacity;
  m.selfCapacity = h.selfCapacity;
  m.dt = R(dt);
  // model.hpp:141-142: fp32 stops at 1e-6, fp64 at 1e-7.
  m.tolerance = sizeof(R) == sizeof(float) ? R(1e-6) : R(1e-7);
  m.alpha = R(0.9);
  m.gamma = R(0.99);
  m.betaLinear = R(1e7);
  m.betaAngular = R(1e5);
  for (int k = 0; k < 3; ++k)
    m.gravity[k] = R(h.gravity[k]);
  for (int b = 0; b < m.nb; ++b) {
    const auto &s = h.bodies[b];
    m.mass[b] = R(s.mass);
    for (int k = 0; k < 3; ++k) {
      m.inertia[k][b] = R(s.inertia[k]);
      m.x[k][b] = R(s.x[k]);
      m.v[k][b] = R(s.v[k]);
      m.w[k][b] = R(s.w[k]);
    }
    for (int k = 0; k < 4; ++k)
      m.q[k][b] = R(s.q[k]);
    m.colors[b] = h.colors[b];
  }
  for (int j = 0; j < m.nj; ++j) {
    const auto &s = h.joints[j];
    m.ja[j] = s.a;
    m.jb[j] = s.b;
    m.limited[j] = s.limited;
    for (int k = 0; k < 3; ++k) {
      m.ra[k][j] = R(s.ra[k]);
      m.rb[k][j] = R(s.rb[k]);
      m.axisA[k][j] = R(s.axisA[k]);
      m.axisB[k][j] = R(s.axisB[k]);
      m.tangentA[k][j] = R(s.tangentA[k]);
      m.tangentB[k][j] = R(s.tangentB[k]);
    }
    m.lo[j] = R(s.lo);
    m.hi[j] = R(s.hi);
    m.armature[j] = R(s.armature);
    m.damping[j] = R(s.damping);
    m.frictionloss[j] = R(s.frictionloss);
    m.torque[j] = R(s.torque);
    m.kp[j] = R(s.kp);
    m.target[j] = R(s.target);
    m.maxTorque[j] = R(s.maxTorque);
  }
  // Hinge angle of the file state in the batch precision, as resetPose
  // evaluates it (kernel.cuh:407-412).
  for (int j = 0; j < m.nj; ++j) {
    int a = m.ja[j], b = m.jb[j];
    Q4<R> qa{m.q[0][a], m.q[1][a], m.q[2][a], m.q[3][a]};
    Q4<R> qb{m.q[0][b], m.q[1][b], m.q[2][b], m.q[3][b]};
    m.originalAngle[j] = hingeAngle(qa, qb, V3<R>{m.axisA[0][j], m.axisA[1][j], m.axisA[2][j]},
                                    V3<R>{m.tangentA[0][j], m.tangentA[1][j], m.tangentA[2][j]},
                                    V3<R>{m.tangentB[0][j], m.tangentB[1][j], m.tangentB[2][j]});
  }
  for (size_t i = 0; i < h.adjacencyStart.size(); ++i)
    m.adjStart[i] = h.adjacencyStart[i];
  for (size_t i = 0; i < h.adjacency.size(); ++i) {
    m.adj[i] = h.adjacency[i];
    m.adjPacked[i] = m.adj[i] | (m.ja[m.adj[i]] << 8) | (m.jb[m.adj[i]] << 16);
  }
  // Default colour schedule: dynamic bodies of colour 0, then of colour 1,
  // each in index order.
  int pos = 0;
  m.colorStart[0] = 0;
  for (int c = 0; c < 2; ++c) {
    for (int b = 0; b < m.nb; ++b)
      if (m.mass[b] > 0 && m.colors[b] == c)
        m.order[pos++] = b;
    m.colorStart[c + 1] = pos;
  }
  for (int s = 0; s < m.ns; ++s) {
    const auto &sh = h.shapes[s];
    m.sbody[s] = sh.body;
    m.stype[s] = sh.type;
    m.sground[s] = sh.ground;
    m.soffset[s] = sh.offset;
    m.scount[s] = sh.count;
    for (int k = 0; k < 3; ++k) {
      m.center[k][s] = R(sh.center[k]);
      m.size[k][s] = R(sh.size[k]);
      m.interior[k][s] = R(sh.interior[k]);
    }
    for (int k = 0; k < 4; ++k)
      m.sq[k][s] = R(sh.q[k]);
    m.sfriction[s] = R(sh.friction);
    m.radius[s] = R(sh.radius);
    const bool pointSet = (sh.type == 1 || sh.type == 3) && sh.count >= 1 && sh.count <= kCachedPoints;
    m.sflags[s] = (h.ground && sh.ground ? 1 : 0) | (pointSet ? 2 : 0);
    for (int k = 0; k < kCachedPoints; ++k)
      for (int c = 0; c < 3; ++c)
        m.spts[k][c][s] = pointSet && k < sh.count ? R(h.points[3 * (sh.offset + k) + c]) : R(0);
  }
  for (int p = 0; p < m.np; ++p) {
    m.pa[p] = h.pairs[p].a;
    m.pb[p] = h.pairs[p].b;
    m.pfriction[p] = R(h.pairs[p].friction);
  }
  // Levels of the Newton-Euler tree: each body a child of at most one hinge,
  // and no body used as a parent before the hinge that makes it a child.
  {
    std::vector<int> parentOf(m.nb, -1);
    std::vector<char> usedAsParent(m.nb, 0);
    bool tree = true;
    int deepest = 0;
    static_assert(kMaxModelJoints <= 32, "a body's child hinges fit one word");
    for (int b = 0; b < m.nb; ++b) {
      m.bodyLevel[b] = 0;
      m.childHinges[b] = 0;
    }
    for (int j = 0; j < m.nj; ++j) {
      const int a = m.ja[j], b = m.jb[j];
      m.childHinges[a] |= 1u << j;
      if (parentOf[b] >= 0 || usedAsParent[b])
        tree = false;
      parentOf[b] = j;
      usedAsParent[a] = 1;
      m.bodyLevel[b] = m.bodyLevel[a] + 1;
      m.jointLevel[j] = m.bodyLevel[b];
      deepest = std::max(deepest, m.bodyLevel[b]);
    }
    m.jointLevels = tree ? deepest : 0;
  }
  return m;
}

struct BatchBase {
  virtual ~BatchBase() = default;
  HostModel host;
  std::vector<std::string> names;
  int count = 0, device = 0, fpBits = 32, contactCapacity = 0;
  long long blobBytes = 0;
  virtual void reset(const unsigned char *, const void *, const void *, const void *,
                     hipStream_t) = 0;
  virtual void step(const void *, const void *, int, double, double, hipStream_t) = 0;
  virtual void stepMotor(const void *, const void *, hipStream_t) = 0;
  virtual void advanceHeld(int, hipStream_t) = 0;
  virtual void state(void *, void *, void *, hipStream_t) = 0;
  virtual void contactForces(int, void *, hipStream_t) = 0;
  virtual void selfContactStats(void *, hipStream_t) = 0;
  virtual void contactCounts(void *, hipStream_t) = 0;
  virtual void generalizedLoads(const void *, void *, hipStream_t) = 0;
  virtual void reference(const void *, const void *, int, double, double, void *, void *,
                         void *) = 0;
  virtual void referenceNoAlloc(const void *, const void *, int, double, double, void *, void *,
                                void *) = 0;
  virtual void layout(long long *out) const = 0;
  virtual void exportState(void *, hipStream_t) = 0;
  virtual void importState(const void *, hipStream_t) = 0;
  virtual void taskTargets(const DuckTask &, const void *, const void *, const long long *,
                           const void *, void *, void *, hipStream_t) = 0;
  virtual void task(const DuckTask &, int, const TaskBuffers &, hipStream_t) = 0;
  virtual void taskResetInputs(const DuckTask &, const unsigned char *, const void *, const void *,
                               const long long *, int, double, const void *, void *, void *,
                               void *, hipStream_t) = 0;
  virtual void servo(const DuckServo &, const ServoBuffers &, hipStream_t) = 0;
  virtual void servoSubstep(const DuckServo &, const DuckServoSubstep &, hipStream_t) = 0;
  virtual void kernelInfo(int which, long long *out) = 0;
};

template <class R, int B, int J, int CG, int CS, int L, int PL = defaultSolveLanes(L)>
class Batch final : public BatchBase {
  using State = EnvState<R, B, J, CG, CS>;
  static constexpr int G = 64 / L;
  DeviceModel<R> *dModel = nullptr;
  Frames<R, B, J> *dFrames = nullptr; // the model's solve-time view (framesKernel)
  V3<R> *dPoints = nullptr;
  unsigned char *dStates = nullptr;
  hipEvent_t ready = nullptr;
  void *dScratch = nullptr; // this device's `scratch`
  // Whether an environment's masses, inertia or friction may differ from the
  // model's (a reset with per-env extensions, an imported state): then every
  // launch reads them from the states, else it takes the model's.
  bool customBodies = false;

  void wait(hipStream_t s) { hipCheck(hipStreamWaitEvent(s, ready, 0), "hipStreamWaitEvent"); }
  void record(hipStream_t s) { hipCheck(hipEventRecord(ready, s), "hipEventRecord"); }
  void launched(const char *what) { hipCheck(hipGetLastError(), what); }
  static int blocks64(int n) { return (n + 63) / 64; }
  // The float MicroDuck-sized batch has a step compiled without body-pair
  // code, launched for models that have none.
  static constexpr bool kPairless = sizeof(R) == sizeof(float) && L == 16;

  void advance(unsigned char *states, int n, const void *targets, const void *forces,
               const void *motor, int substeps, double kp, double limit, hipStream_t s,
               int mode = -1) {
    if (mode < 0)
      mode = motor != nullptr ? kMotorControls : kTargetControls;
    StepArgs args{dModel, dFrames, dPoints, states, blobBytes, n, targets, forces, motor,
                  substeps, mode, kp, limit,
                  int(host.bodies.size()), int(host.joints.size()), int(host.shapes.size()),
                  int(host.pairs.size()), states == dStates && customBodies ? 1 : 0};
    if constexpr (kPairless) {
      if (host.pairs.empty())
        advanceKernel<R, B, J, CG, CS, L, PL, false><<<(n + G - 1) / G, 64, 0, s>>>(args);
      else
        advanceKernel<R, B, J, CG, CS, L, PL><<<(n + G - 1) / G, 64, 0, s>>>(args);
    } else {
      advanceKernel<R, B, J, CG, CS, L, PL><<<(n + G - 1) / G, 64, 0, s>>>(args);
    }
    launched("advanceKernel");
  }

public:
  Batch(HostModel &&model, int n, double dt, int iterations, int gpu) {
    host = std::move(model);
    count = n;
    device = gpu;
    fpBits = sizeof(R) * 8;
    contactCapacity = host.groundCapacity + host.selfCapacity;
    blobBytes = (sizeof(State) + 127) / 128 * 128;
    for (auto &j : host.joints)
      names.push_back(j.name);
    DeviceGuard guard(device);
    DeviceModel<R> packed = pack<R>(host, dt, iterations);
    std::vector<V3<R>> pts(std::max<size_t>(1, host.points.size() / 3));
    for (size_t i = 0; i < host.points.size() / 3; ++i)
      pts[i] = V3<R>{R(host.points[3 * i]), R(host.points[3 * i + 1]), R(host.points[3 * i + 2])};
    try {
      hipCheck(hipMalloc(&dModel, sizeof(DeviceModel<R>)), "hipMalloc(model)");
      hipCheck(hipMalloc(&dPoints, pts.size() * sizeof(V3<R>)), "hipMalloc(points)");
      hipCheck(hipMalloc(&dStates, size_t(blobBytes) * count), "hipMalloc(state)");
      hipCheck(hipMemcpy(dModel, &packed, sizeof(packed), hipMemcpyHostToDevice), "upload model");
      hipCheck(hipMalloc(&dFrames, sizeof(Frames<R, B, J>)), "hipMalloc(frames)");
      hipCheck(hipMemset(dFrames, 0, sizeof(Frames<R, B, J>)), "hipMemset(frames)");
      framesKernel<R, B, J><<<1, 64, 0, 0>>>(dModel, dFrames);
      launched("framesKernel");
      hipCheck(hipMemcpy(dPoints, pts.data(), pts.size() * sizeof(V3<R>), hipMemcpyHostToDevice),
               "upload points");
      hipCheck(hipMemset(dStates, 0, size_t(blobBytes) * count), "hipMemset(state)");
      initializeKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, 0>>>(dModel, dStates, blobBytes,
                                                                        count);
      launched("initializeKernel");
      hipCheck(hipDeviceSynchronize(), "initialize");
      hipCheck(hipEventCreateWithFlags(&ready, hipEventDisableTiming), "hipEventCreate");
      dScratch = referenceScratch(device);
      record(0);
    } catch (...) {
      release();
      throw;
    }
  }
  void release() {
    if (ready) {
      (void)hipEventSynchronize(ready);
      (void)hipEventDestroy(ready);
      ready = nullptr;
    }
    if (dStates)
      (void)hipFree(dStates);
    if (dPoints)
      (void)hipFree(dPoints);
    if (dModel)
      (void)hipFree(dModel);
    if (dFrames)
      (void)hipFree(dFrames);
    dStates = nullptr;
    dPoints = nullptr;
    dModel = nullptr;
    dFrames = nullptr;
  }
  ~Batch() override {
    try {
      DeviceGuard guard(device);
      release();
    } catch (...) {
    }
  }

  void reset(const unsigned char *mask, const void *q, const void *root, const void *ext,
             hipStream_t s) override {
    DeviceGuard guard(device);
    // joint-indexed buffers of a model without hinges are empty (may be null)
    const bool noJoints = host.joints.empty();
    require(mask && (q || noJoints) && root, "reset: null buffer");
    wait(s);
    resetKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(
        dModel, dStates, blobBytes, count, mask, static_cast<const R *>(q),
        static_cast<const R *>(root), static_cast<const R *>(ext));
    launched("resetKernel");
    if (ext)
      customBodies = true;
    record(s);
  }
  void step(const void *target, const void *force, int substeps, double kp, double limit,
            hipStream_t s) override {
    DeviceGuard guard(device);
    require((target || host.joints.empty()) && force, "step: null buffer");
    // extension.cu:290-294: zero limit = uncapped; negative/non-finite invalid.
    require(substeps > 0 && kp >= 0 && std::isfinite(kp) && limit >= 0 && std::isfinite(limit),
            "Invalid controls");
    wait(s);
    advance(dStates, count, target, force, nullptr, substeps, kp, limit, s);
    record(s);
  }
  void stepMotor(const void *motor, const void *force, hipStream_t s) override {
    DeviceGuard guard(device);
    require((motor || host.joints.empty()) && force, "step_motor: null buffer");
    wait(s);
    advance(dStates, count, nullptr, force, motor, 1, 0, 0, s);
    record(s);
  }
  void advanceHeld(int substeps, hipStream_t s) override {
    DeviceGuard guard(device);
    require(substeps > 0, "Invalid controls");
    wait(s);
    advance(dStates, count, nullptr, nullptr, nullptr, substeps, 0, 0, s, kHeldControls);
    record(s);
  }
  void state(void *bodies, void *joints, void *diag, hipStream_t s) override {
    DeviceGuard guard(device);
    require(bodies && (joints || host.joints.empty()) && diag, "state: null buffer");
    wait(s);
    snapshotKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(
        dModel, dStates, blobBytes, count, static_cast<R *>(bodies), static_cast<R *>(joints),
        static_cast<R *>(diag));
    launched("snapshotKernel");
    record(s);
  }
  void contactForces(int groundOnly, void *out, hipStream_t s) override {
    DeviceGuard guard(device);
    require(out, "contact_forces: null buffer");
    wait(s);
    contactForcesKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(
        dModel, dStates, blobBytes, count, groundOnly, static_cast<R *>(out));
    launched("contactForcesKernel");
    record(s);
  }
  void selfContactStats(void *out, hipStream_t s) override {
    DeviceGuard guard(device);
    require(out, "self_contact_stats: null buffer");
    wait(s);
    selfContactStatsKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(
        dModel, dStates, blobBytes, count, static_cast<R *>(out));
    launched("selfContactStatsKernel");
    record(s);
  }
  void contactCounts(void *out, hipStream_t s) override {
    DeviceGuard guard(device);
    require(out, "contact_counts: null buffer");
    wait(s);
    contactCountsKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(dStates, blobBytes, count,
                                                                        static_cast<R *>(out));
    launched("contactCountsKernel");
    record(s);
  }
  void generalizedLoads(const void *offset, void *out, hipStream_t s) override {
    DeviceGuard guard(device);
    require(offset && (out || host.joints.empty()), "generalized_loads: null buffer");
    wait(s);
    generalizedLoadsKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(
        dModel, dStates, blobBytes, count, static_cast<const R *>(offset), static_cast<R *>(out));
    launched("generalizedLoadsKernel");
    record(s);
  }
  // Reals of duck_reference's device inputs and outputs: target, force,
  // bodies, joints, diag.
  size_t referenceIoCount() const {
    const int nb = host.bodies.size(), nj = host.joints.size();
    return size_t(nj) + 3 + size_t(nb) * 13 + size_t(nj) * 2 + 6;
  }
  // One environment from the model file's state (extension.cu:385-415) in
  // `state` (blobBytes of device memory) with its inputs and outputs in `io`
  // (referenceIoCount() device reals); synchronous, on the null stream.
  void referenceIn(unsigned char *state, R *io, const void *target, const void *force,
                   int substeps, double kp, double limit, void *bodies, void *joints, void *diag) {
    require(target && force && bodies && joints && diag && substeps > 0,
            "Invalid CPU reference inputs");
    const int nb = host.bodies.size(), nj = host.joints.size();
    R *dTarget = io, *dForce = io + nj, *dB = dForce + 3, *dJ = dB + nb * 13, *dD = dJ + nj * 2;
    hipCheck(hipMemcpy(dTarget, target, nj * sizeof(R), hipMemcpyHostToDevice), "upload");
    hipCheck(hipMemcpy(dForce, force, 3 * sizeof(R), hipMemcpyHostToDevice), "upload");
    zeroWordsKernel<<<(blobBytes / 4 + 63) / 64, 64, 0, 0>>>(reinterpret_cast<unsigned *>(state),
                                                             blobBytes / 4);
    launched("zeroWordsKernel");
    initializeKernel<R, B, J, CG, CS><<<1, 64, 0, 0>>>(dModel, state, blobBytes, 1);
    launched("initializeKernel");
    // extension.cu:403-410 sets force, kp, limit and target only; the
    // model's torque/friction/damping are already in place.
    advance(state, 1, dTarget, dForce, nullptr, substeps, kp, limit, 0);
    snapshotKernel<R, B, J, CG, CS><<<1, 64, 0, 0>>>(dModel, state, blobBytes, 1, dB, dJ, dD);
    launched("snapshotKernel");
    hipCheck(hipMemcpy(bodies, dB, nb * 13 * sizeof(R), hipMemcpyDeviceToHost), "download");
    hipCheck(hipMemcpy(joints, dJ, nj * 2 * sizeof(R), hipMemcpyDeviceToHost), "download");
    hipCheck(hipMemcpy(diag, dD, 6 * sizeof(R), hipMemcpyDeviceToHost), "download");
  }
  void reference(const void *target, const void *force, int substeps, double kp, double limit,
                 void *bodies, void *joints, void *diag) override {
    DeviceGuard guard(device);
    require(target && force && bodies && joints && diag && substeps > 0,
            "Invalid CPU reference inputs");
    unsigned char *state = nullptr;
    R *buf = nullptr;
    try {
      hipCheck(hipMalloc(&state, blobBytes), "hipMalloc(reference state)");
      hipCheck(hipMalloc(&buf, referenceIoCount() * sizeof(R)), "hipMalloc(reference io)");
      referenceIn(state, buf, target, force, substeps, kp, limit, bodies, joints, diag);
    } catch (...) {
      if (state)
        (void)hipFree(state);
      if (buf)
        (void)hipFree(buf);
      throw;
    }
    hipCheck(hipFree(state), "hipFree");
    hipCheck(hipFree(buf), "hipFree");
  }
  // duck_reference with the blob and the inputs/outputs in this device's
  // `scratch` (blob first, 256-byte aligned, then the reals): no allocation.
  void referenceNoAlloc(const void *target, const void *force, int substeps, double kp,
                        double limit, void *bodies, void *joints, void *diag) override {
    DeviceGuard guard(device);
    const size_t need = size_t(blobBytes) + referenceIoCount() * sizeof(R);
    if (need > kReferenceScratchBytes)
      throw DuckError(DUCK_ERR_ARGUMENT,
                      "reference scratch: this model needs " + std::to_string(need) +
                          " bytes of the library's " + std::to_string(kReferenceScratchBytes));
    require(dScratch != nullptr, "reference scratch: no device address");
    std::lock_guard<std::mutex> lock(referenceScratchLock(device));
    unsigned char *base = static_cast<unsigned char *>(dScratch);
    referenceIn(base, reinterpret_cast<R *>(base + blobBytes), target, force, substeps, kp, limit,
                bodies, joints, diag);
  }
  void taskTargets(const DuckTask &t, const void *actions, const void *reference,
                   const long long *episode, const void *commands, void *clamped, void *target,
                   hipStream_t s) override {
    DeviceGuard guard(device);
    require(actions && clamped && target, "task targets: null buffer");
    const int nj = host.joints.size();
    taskTargetsKernel<R><<<blocks64(count * nj), 64, 0, s>>>(
        t, count, nj, static_cast<const R *>(actions), static_cast<const R *>(reference), episode,
        static_cast<const R *>(commands), static_cast<R *>(clamped), static_cast<R *>(target));
    launched("taskTargetsKernel");
  }
  void taskResetInputs(const DuckTask &t, const unsigned char *mask, const void *jointDraws,
                       const void *rootDraws, const long long *selected, int direction,
                       double speed, const void *commands, void *q, void *roots,
                       void *commandsOut, hipStream_t s) override {
    DeviceGuard guard(device);
    const int nj = host.joints.size();
    taskResetInputsKernel<R><<<blocks64(count * std::max(nj, 1)), 64, 0, s>>>(
        t, count, nj, mask, static_cast<const R *>(jointDraws), static_cast<const R *>(rootDraws),
        selected, direction, R(speed), static_cast<const R *>(commands), static_cast<R *>(q),
        static_cast<R *>(roots), static_cast<R *>(commandsOut));
    launched("taskResetInputsKernel");
  }
  void task(const DuckTask &t, int mode, const TaskBuffers &io, hipStream_t s) override {
    DeviceGuard guard(device);
    wait(s);
    constexpr int TE = taskEnvsPerBlock<State>();
    taskKernel<R, B, J, CG, CS><<<(count + TE - 1) / TE, 64, 0, s>>>(t, mode, dModel, dStates, blobBytes,
                                                                count, io);
    launched("taskKernel");
    record(s);
  }
  void servoSubstep(const DuckServo &p, const DuckServoSubstep &io, hipStream_t s) override {
    DeviceGuard guard(device);
    const int nb = host.bodies.size();
    require(nb >= 2, "servo substep: the model needs a root body (body 1)");
    require(io.num_feet >= 0 && io.num_feet <= DUCK_MAX_FEET, "servo substep: invalid foot count");
    ServoArgs<R> sv{};
    sv.p = p;
    sv.cursor = io.cursor;
    sv.target = static_cast<const R *>(io.target);
    sv.history = static_cast<R *>(io.history);
    sv.initialized = io.initialized;
    sv.rootOffset = static_cast<const R *>(io.root_offset);
    sv.previousMotor = static_cast<R *>(io.previous_motor);
    sv.previousApplied = static_cast<R *>(io.previous_applied);
    sv.motor = static_cast<R *>(io.motor);
    sv.supply = static_cast<R *>(io.supply);
    sv.selfContacts = static_cast<R *>(io.self_contacts);
    sv.selfPenetration = static_cast<R *>(io.self_penetration);
    // root frame = q1 * conj(root principal rotation) (bam_env.py:64, 130-132)
    sv.rootInv[0] = R(io.root_principal_quat[0]);
    for (int k = 1; k < 4; ++k)
      sv.rootInv[k] = -R(io.root_principal_quat[k]);
    sv.numFeet = io.num_feet;
    for (int f = 0; f < io.num_feet; ++f) {
      require(io.foot_bodies[f] >= 0 && io.foot_bodies[f] < nb, "servo substep: invalid foot body");
      sv.feet[f] = io.foot_bodies[f];
      for (int k = 0; k < 3; ++k)
        sv.sites[f][k] = R(io.foot_sites[f][k]);
    }
    sv.gravity = static_cast<R *>(io.gravity);
    sv.angularVelocity = static_cast<R *>(io.angular_velocity);
    sv.linearVelocity = static_cast<R *>(io.linear_velocity);
    sv.originVelocity = static_cast<R *>(io.origin_velocity);
    sv.footForces = static_cast<R *>(io.foot_forces);
    sv.sitePositions = static_cast<R *>(io.site_positions);
    sv.siteVelocities = static_cast<R *>(io.site_velocities);
    sv.airTime = static_cast<R *>(io.air_time);
    sv.contactTime = static_cast<R *>(io.contact_time);
    sv.meanVelocity = static_cast<R *>(io.mean_velocity);
    require(!io.mean_velocity || (io.mean_velocity_alpha >= 0 && io.mean_velocity_alpha <= 1),
            "servo substep: mean_velocity_alpha outside [0, 1]");
    sv.meanAlpha = R(io.mean_velocity_alpha);
    StepArgs args{dModel, dFrames, dPoints, dStates, blobBytes, count, nullptr, nullptr, nullptr,
                  1, kMotorControls, 0, 0,
                  nb, int(host.joints.size()), int(host.shapes.size()), int(host.pairs.size()),
                  customBodies ? 1 : 0};
    wait(s);
    if constexpr (kPairless) {
      if (host.pairs.empty())
        servoStepKernel<R, B, J, CG, CS, L, PL, false><<<(count + G - 1) / G, 64, 0, s>>>(args, sv);
      else
        servoStepKernel<R, B, J, CG, CS, L, PL><<<(count + G - 1) / G, 64, 0, s>>>(args, sv);
    } else {
      servoStepKernel<R, B, J, CG, CS, L, PL><<<(count + G - 1) / G, 64, 0, s>>>(args, sv);
    }
    launched("servoStepKernel");
    record(s);
  }
  void servo(const DuckServo &p, const ServoBuffers &io, hipStream_t s) override {
    DeviceGuard guard(device);
    wait(s);
    servoKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(p, dModel, dStates, blobBytes,
                                                                 count, io);
    launched("servoKernel");
    record(s);
  }
  void layout(long long *out) const override;
  // Resources of the kernel this batch's duck_step (which = DUCK_KERNEL_STEP)
  // or duck_servo_substep (DUCK_KERNEL_SERVO_SUBSTEP) launches -- the build
  // without body-pair code for a model without pairs: VGPRs, static LDS and
  // scratch per lane from the code object, resident workgroups per CU from
  // the runtime's occupancy calculator, lanes and environments per
  // workgroup, and workgroups per launch.
  void kernelInfo(int which, long long *out) override {
    DeviceGuard guard(device);
    require(which == DUCK_KERNEL_STEP || which == DUCK_KERNEL_SERVO_SUBSTEP,
            "kernel_info: unknown kernel");
    const bool pairless = kPairless && host.pairs.empty();
    const void *fn = nullptr;
    if (which == DUCK_KERNEL_STEP)
      fn = reinterpret_cast<const void *>(&advanceKernel<R, B, J, CG, CS, L, PL>);
    else
      fn = reinterpret_cast<const void *>(&servoStepKernel<R, B, J, CG, CS, L, PL>);
    if constexpr (kPairless) {
      if (pairless && which == DUCK_KERNEL_STEP)
        fn = reinterpret_cast<const void *>(&advanceKernel<R, B, J, CG, CS, L, PL, false>);
      if (pairless && which == DUCK_KERNEL_SERVO_SUBSTEP)
        fn = reinterpret_cast<const void *>(&servoStepKernel<R, B, J, CG, CS, L, PL, false>);
    }
    hipFuncAttributes a{};
    hipCheck(hipFuncGetAttributes(&a, fn), "hipFuncGetAttributes");
    int perCu = 0;
    hipCheck(hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu, fn, 64, 0),
             "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    const long long v[7] = {a.numRegs, static_cast<long long>(a.sharedSizeBytes),
                            static_cast<long long>(a.localSizeBytes), perCu, 64, G,
                            (count + G - 1) / G};
    for (int i = 0; i < 7; ++i)
      out[i] = v[i];
  }
  void exportState(void *dst, hipStream_t s) override {
    DeviceGuard guard(device);
    require(dst, "export_state: null buffer");
    wait(s);
    hipCheck(hipMemcpyAsync(dst, dStates, size_t(blobBytes) * count, hipMemcpyDeviceToDevice, s),
             "export_state");
    record(s);
  }
  void importState(const void *src, hipStream_t s) override {
    DeviceGuard guard(device);
    require(src, "import_state: null buffer");
    wait(s);
    hipCheck(hipMemcpyAsync(dStates, src, size_t(blobBytes) * count, hipMemcpyDeviceToDevice, s),
             "import_state");
    checkStampsKernel<R, B, J, CG, CS><<<blocks64(count), 64, 0, s>>>(dModel, dStates, blobBytes, count);
    launched("checkStampsKernel");
    customBodies = true;
    record(s);
  }
};

#define DUCK_OFF(T, f) static_cast<long long>(offsetof(T, f))
template <class R, int B, int J, int CG, int CS, int L, int PL>
void Batch<R, B, J, CG, CS, L, PL>::layout(long long *o) const {
  using S = EnvState<R, B, J, CG, CS>;
  using GC = GroundContact<R>;
  using SC = SelfContact<R>;
  const long long v[] = {
      B, J, CG, CS, sizeof(R), blobBytes, static_cast<long long>(headerBytes<S>()),
      DUCK_OFF(S, x), DUCK_OFF(S, q), DUCK_OFF(S, v), DUCK_OFF(S, w), DUCK_OFF(S, mass),
      DUCK_OFF(S, inertia), DUCK_OFF(S, force), DUCK_OFF(S, lambda), DUCK_OFF(S, penalty),
      DUCK_OFF(S, lambdaF), DUCK_OFF(S, penaltyF), DUCK_OFF(S, target), DUCK_OFF(S, kp),
      DUCK_OFF(S, maxTorque), DUCK_OFF(S, torque), DUCK_OFF(S, frictionloss),
      DUCK_OFF(S, damping), DUCK_OFF(S, diag), DUCK_OFF(S, friction), DUCK_OFF(S, failed),
      DUCK_OFF(S, ngc), DUCK_OFF(S, nsc), DUCK_OFF(S, colors), DUCK_OFF(S, colorCount),
      DUCK_OFF(S, gc), static_cast<long long>(sizeof(GC)), DUCK_OFF(S, sc),
      static_cast<long long>(sizeof(SC)), DUCK_OFF(GC, id), DUCK_OFF(GC, local),
      DUCK_OFF(GC, anchor), DUCK_OFF(GC, c0), DUCK_OFF(GC, lambda), DUCK_OFF(GC, penalty),
      DUCK_OFF(SC, id), DUCK_OFF(SC, local), DUCK_OFF(SC, localB), DUCK_OFF(SC, t1),
      DUCK_OFF(SC, t2), DUCK_OFF(SC, n), DUCK_OFF(SC, c0), DUCK_OFF(SC, friction),
      DUCK_OFF(SC, lambda), DUCK_OFF(SC, penalty)};
  static_assert(sizeof(v) / sizeof(v[0]) == 51, "layout descriptor has 51 entries");
  for (int i = 0; i < 51; ++i)
    o[i] = v[i];
}
#undef DUCK_OFF

const char *kMicroDuckJoints[14] = {
    "left_hip_yaw",    "left_hip_roll",  "left_hip_pitch", "left_knee",
    "left_ankle",      "neck_pitch",     "head_pitch",     "head_yaw",
    "head_roll",       "right_hip_yaw",  "right_hip_roll", "right_hip_pitch",
    "right_knee",      "right_ankle"};

// MicroDuck-sized models (16 bodies and 14 hinges, the reference's
// MicroDuckState, kernel.cuh:1098): float runs 4 environments per wave with two lanes
// per block solve (16 lanes per env); double runs 8 environments per wave
// with one lane per block solve, which keeps the reference's accumulation
// order (DUCK_FLAG_SPLIT selects the float layout for double too).  Four
// lanes per block solve (32 lanes per env, 20 KB of LDS per workgroup)
// would let two waves share a SIMD only below 256 registers per lane, which
// this kernel exceeds; with register spills it measured slower.
template <class R>
BatchBase *makeBatch(HostModel &&m, int n, double dt, int iterations, int device, bool split) {
  const int nb = m.bodies.size(), nj = m.joints.size(), ns = m.shapes.size(),
            np = m.pairs.size();
  if (nb <= 16 && nj <= 14 && ns <= 16 && np <= 8 && m.groundCapacity <= 64) {
    if constexpr (sizeof(R) == sizeof(double))
      if (!split)
        return new Batch<R, 16, 14, 64, 8, 8>(std::move(m), n, dt, iterations, device);
    return new Batch<R, 16, 14, 64, 8, 16>(std::move(m), n, dt, iterations, device);
  }
  // The generic state: 32 bodies and hinges, 4 ground contacts for each of
  // up to 32 shapes and one per body-contact pair (the reference's
  // BasicState<32, 32, 160>, kernel.cuh:365, holds the sum of both).
  // Float (and float64 with DUCK_FLAG_SPLIT): four lanes per block solve;
  // float64: one lane per block solve, the reference's accumulation order.
  if (m.groundCapacity > 128 || m.selfCapacity > 32)
    throw DuckError(DUCK_ERR_MODEL, "Model exceeds selected state contact capacity");
  if constexpr (sizeof(R) == sizeof(double))
    if (!split)
      return new Batch<R, 32, 32, 128, 32, 32, 1>(std::move(m), n, dt, iterations, device);
  return new Batch<R, 32, 32, 128, 32, 32>(std::move(m), n, dt, iterations, device);
}

// The model checks of the selected backend after loadModel's flattening
// checks: the specialized state's capacities (model.hpp:30-40 with
// MicroDuckState<16, 14, 64>, kernel.cuh:1098; std::invalid_argument, a
// ValueError in Python), then its exact layout (extension.cu:225-236;
// TORCH_CHECK, a RuntimeError).  The generic state's capacities (32 bodies
// and joints, pairs + 4 per ground shape <= 160) follow from loadModel's
// 32-body/joint/shape/pair limit.
void checkBackend(const HostModel &m, unsigned flags) {
  if (!(flags & DUCK_FLAG_SPECIALIZED))
    return;
  if (m.bodies.size() > 16 || m.joints.size() > 14)
    throw std::invalid_argument("Model exceeds selected state body/joint capacity");
  if (m.groundCapacity + m.selfCapacity > 64)
    throw std::invalid_argument("Model exceeds selected state contact capacity");
  require(m.bodies.size() == 16 && m.joints.size() == 14,
          "MicroDuck specialized backend requires 16 bodies and 14 hinges");
  for (int i = 0; i < 14; ++i) {
    std::string label = m.joints[i].name;
    if (label.rfind("robot/", 0) == 0)
      label = label.substr(6);
    require(label == kMicroDuckJoints[i], "Unsupported MicroDuck joint layout");
  }
}

template <class F> int guarded(F &&f) {
  try {
    f();
    return DUCK_OK;
  } catch (const DuckError &e) {
    g_lastError = e.what();
    return e.code;
  } catch (const std::invalid_argument &e) {
    // model.hpp:5-8 checks (pybind11 maps them to ValueError)
    g_lastError = e.what();
    return DUCK_ERR_MODEL;
  } catch (const std::exception &e) {
    // Solver::load errors (pybind11 maps them to RuntimeError)
    g_lastError = e.what();
    return DUCK_ERR_RUNTIME;
  }
}
BatchBase *as(void *h) {
  if (!h)
    throw DuckError(DUCK_ERR_ARGUMENT, "null batch handle");
  return static_cast<BatchBase *>(h);
}
hipStream_t st(void *s) { return static_cast<hipStream_t>(s); }

// ---- explicit-sequential step (duck_sequential_step) ----

// `steps` steps of environment i, whose record starts at records + offset[i];
// an environment stops at its first fault.
__global__ __launch_bounds__(64) void sequentialStepKernel(unsigned char *records,
                                                           const long long *offset, int n,
                                                           int steps) {
  const int i = blockIdx.x * 64 + threadIdx.x;
  if (i >= n)
    return;
  seq::Env e(records + offset[i]);
  for (int s = 0; s < steps && e.r->status == DUCK_SEQ_OK; ++s)
    e.step();
}

// The same with one environment per workgroup and its record staged in LDS
// (dynamic shared memory of the largest record's size): the workgroup copies
// the record in, its first thread runs the steps on the LDS copy, and the
// workgroup copies it back.  Records are whole 256-byte multiples.
__global__ __launch_bounds__(64) void sequentialStepLdsKernel(unsigned char *records,
                                                              const long long *offset, int n,
                                                              long long total, int steps) {
  extern __shared__ uint4 seqRecord[];
  const int i = blockIdx.x;
  const long long begin = offset[i], end = i + 1 < n ? offset[i + 1] : total;
  const int chunks = int((end - begin) / 16);
  uint4 *global = reinterpret_cast<uint4 *>(records + begin);
  for (int k = threadIdx.x; k < chunks; k += 64)
    seqRecord[k] = global[k];
  __syncthreads();
  if (threadIdx.x == 0) {
    seq::Env e(reinterpret_cast<unsigned char *>(seqRecord));
    for (int s = 0; s < steps && e.r->status == DUCK_SEQ_OK; ++s)
      e.step();
  }
  __syncthreads();
  for (int k = threadIdx.x; k < chunks; k += 64)
    global[k] = seqRecord[k];
}
// Records up to this size take the LDS kernel when the batch has at most
// kSequentialLdsEnvs environments: one environment per workgroup measured
// 12 % faster per step than the device-memory kernel for one environment,
// and slower from a few hundred on (where 64 environments share a wave).
constexpr long long kSequentialLdsBytes = 64 << 10;
constexpr int kSequentialLdsEnvs = 64;

// The device buffers of one device, reused and grown across calls; calls on
// one device take turns on them.
struct SequentialBuffers {
  std::mutex lock;
  unsigned char *records = nullptr;
  long long *offsets = nullptr;
  size_t recordBytes = 0, offsetCount = 0;
};
SequentialBuffers &sequentialBuffers(int device) {
  static std::mutex guard;
  static std::vector<std::unique_ptr<SequentialBuffers>> all;
  std::lock_guard<std::mutex> lock(guard);
  require(device >= 0 && device < 1024, "sequential step: invalid device");
  if (device >= int(all.size()))
    all.resize(device + 1);
  if (!all[device])
    all[device] = std::make_unique<SequentialBuffers>();
  return *all[device];
}

void sequentialStep(DuckSeqEnv *envs, int n, int steps, int device) {
  require(envs != nullptr && n > 0 && steps > 0, "sequential step: no environments or steps");
  int devices = 0;
  hipCheck(hipGetDeviceCount(&devices), "hipGetDeviceCount");
  require(device >= 0 && device < devices, "sequential step: invalid device");
  std::vector<unsigned char> image;
  std::vector<long long> offsets;
  try {
    for (int i = 0; i < n; ++i)
      seq::checkSequential(envs[i], steps);
    seq::packSequential(envs, n, image, offsets);
  } catch (const seq::SeqError &e) {
    throw DuckError(DUCK_ERR_ARGUMENT, e.what());
  }
  const size_t total = image.size();
  DeviceGuard guard(device);
  SequentialBuffers &buf = sequentialBuffers(device);
  std::lock_guard<std::mutex> lock(buf.lock);
  if (total > buf.recordBytes) {
    if (buf.records)
      hipCheck(hipFree(buf.records), "hipFree(sequential records)");
    buf.records = nullptr;
    buf.recordBytes = 0;
    hipCheck(hipMalloc(&buf.records, total), "hipMalloc(sequential records)");
    buf.recordBytes = total;
  }
  if (size_t(n) > buf.offsetCount) {
    if (buf.offsets)
      hipCheck(hipFree(buf.offsets), "hipFree(sequential offsets)");
    buf.offsets = nullptr;
    buf.offsetCount = 0;
    hipCheck(hipMalloc(&buf.offsets, sizeof(long long) * n), "hipMalloc(sequential offsets)");
    buf.offsetCount = n;
  }
  hipCheck(hipMemcpy(buf.records, image.data(), total, hipMemcpyHostToDevice), "upload");
  hipCheck(hipMemcpy(buf.offsets, offsets.data(), sizeof(long long) * n, hipMemcpyHostToDevice),
           "upload");
  long long largest = 0;
  for (int i = 0; i < n; ++i)
    largest = std::max(largest, (i + 1 < n ? offsets[i + 1] : (long long)total) - offsets[i]);
  if (largest <= kSequentialLdsBytes && n <= kSequentialLdsEnvs) {
    sequentialStepLdsKernel<<<n, 64, size_t(largest), 0>>>(buf.records, buf.offsets, n,
                                                           (long long)total, steps);
    hipCheck(hipGetLastError(), "sequentialStepLdsKernel");
  } else {
    sequentialStepKernel<<<(n + 63) / 64, 64, 0, 0>>>(buf.records, buf.offsets, n, steps);
    hipCheck(hipGetLastError(), "sequentialStepKernel");
  }
  hipCheck(hipMemcpy(image.data(), buf.records, total, hipMemcpyDeviceToHost), "download");
  seq::unpackSequential(envs, n, image, offsets);
}

} // namespace
} // namespace duckhip

using namespace duckhip;

extern "C" {

const char *duck_last_error(void) { return g_lastError.c_str(); }

int duck_model_info(const char *model_path, unsigned flags, int *out) {
  return guarded([&] {
    require(model_path != nullptr && out != nullptr, "null argument");
    require(!(flags & DUCK_FLAG_SHARED_MEMORY) || (flags & DUCK_FLAG_SPECIALIZED),
            "Shared memory requires the compact MicroDuck backend");
    HostModel m = loadModel(model_path);
    checkBackend(m, flags);
    const int v[] = {int(m.bodies.size()), int(m.joints.size()), int(m.shapes.size()),
                     int(m.pairs.size()), m.groundCapacity, m.selfCapacity};
    for (int i = 0; i < 6; ++i)
      out[i] = v[i];
  });
}

namespace {
// duck_create and duck_create_text: the model from a file or from text, then
// the batch checks and the batch.
int createBatch(const char *source, bool text, int num_envs, double dt, int iterations,
                int device, int fp_bits, unsigned flags, void **out_handle) {
  return guarded([&] {
    require(out_handle != nullptr && source != nullptr, "null argument");
    *out_handle = nullptr;
    // extension.cu:424 checks the shared-memory option before anything else
    require(!(flags & DUCK_FLAG_SHARED_MEMORY) || (flags & DUCK_FLAG_SPECIALIZED),
            "Shared memory requires the compact MicroDuck backend");
    require(num_envs > 0 && num_envs <= 65536 && dt > 0 && std::isfinite(dt) && iterations > 0,
            "Invalid batch parameters");
    require(fp_bits == 32 || fp_bits == 64, "fp_bits must be 32 or 64");
    int devices = 0;
    hipCheck(hipGetDeviceCount(&devices), "hipGetDeviceCount");
    require(device >= 0 && device < devices, "Invalid device index");
    HostModel m = text ? loadModelText(source) : loadModel(source);
    checkBackend(m, flags);
    const bool split = flags & DUCK_FLAG_SPLIT;
    BatchBase *b =
        fp_bits == 64 ? makeBatch<double>(std::move(m), num_envs, dt, iterations, device, split)
                      : makeBatch<float>(std::move(m), num_envs, dt, iterations, device, split);
    *out_handle = b;
  });
}
} // namespace

int duck_create(const char *model_path, int num_envs, double dt, int iterations, int device,
                int fp_bits, unsigned flags, void **out_handle) {
  return createBatch(model_path, false, num_envs, dt, iterations, device, fp_bits, flags,
                     out_handle);
}

int duck_create_text(const char *model_text, int num_envs, double dt, int iterations, int device,
                     int fp_bits, unsigned flags, void **out_handle) {
  return createBatch(model_text, true, num_envs, dt, iterations, device, fp_bits, flags,
                     out_handle);
}

void duck_destroy(void *handle) { delete static_cast<BatchBase *>(handle); }

int duck_dims(void *handle, int *bodies, int *joints, int *contact_capacity) {
  return guarded([&] {
    auto *b = as(handle);
    if (bodies)
      *bodies = b->host.bodies.size();
    if (joints)
      *joints = b->host.joints.size();
    if (contact_capacity)
      *contact_capacity = b->contactCapacity;
  });
}
int duck_num_envs(void *handle) { return handle ? as(handle)->count : 0; }
int duck_fp_bits(void *handle) { return handle ? as(handle)->fpBits : 0; }
long long duck_state_bytes(void *handle) { return handle ? as(handle)->blobBytes : 0; }

const char *duck_joint_name(void *handle, int index) {
  if (!handle)
    return nullptr;
  auto *b = as(handle);
  if (index < 0 || index >= int(b->names.size()))
    return nullptr;
  return b->names[index].c_str();
}

int duck_reset(void *handle, const unsigned char *mask, const void *q, const void *root,
               const void *ext, void *hip_stream) {
  return guarded([&] { as(handle)->reset(mask, q, root, ext, st(hip_stream)); });
}
int duck_step(void *handle, const void *target, const void *force, int substeps, double kp,
              double limit, void *hip_stream) {
  return guarded([&] { as(handle)->step(target, force, substeps, kp, limit, st(hip_stream)); });
}
int duck_step_motor(void *handle, const void *motor, const void *force, void *hip_stream) {
  return guarded([&] { as(handle)->stepMotor(motor, force, st(hip_stream)); });
}
int duck_advance(void *handle, int substeps, void *hip_stream) {
  return guarded([&] { as(handle)->advanceHeld(substeps, st(hip_stream)); });
}
int duck_state(void *handle, void *bodies, void *joints, void *diag, void *hip_stream) {
  return guarded([&] { as(handle)->state(bodies, joints, diag, st(hip_stream)); });
}
int duck_contact_forces(void *handle, int ground_only, void *out, void *hip_stream) {
  return guarded([&] { as(handle)->contactForces(ground_only, out, st(hip_stream)); });
}
int duck_self_contact_stats(void *handle, void *out, void *hip_stream) {
  return guarded([&] { as(handle)->selfContactStats(out, st(hip_stream)); });
}
int duck_contact_counts(void *handle, void *out, void *hip_stream) {
  return guarded([&] { as(handle)->contactCounts(out, st(hip_stream)); });
}
int duck_generalized_loads(void *handle, const void *offset, void *out, void *hip_stream) {
  return guarded([&] { as(handle)->generalizedLoads(offset, out, st(hip_stream)); });
}
int duck_sequential_step(DuckSeqEnv *envs, int num_envs, int steps, int device) {
  return guarded([&] { sequentialStep(envs, num_envs, steps, device); });
}

int duck_kernel_info(void *handle, int which, long long *out) {
  return guarded([&] {
    require(handle != nullptr && out != nullptr, "null argument");
    as(handle)->kernelInfo(which, out);
  });
}

int duck_state_layout(void *handle, long long *out) {
  return guarded([&] {
    require(out != nullptr, "null argument");
    as(handle)->layout(out);
  });
}
int duck_export_state(void *handle, void *dst, void *hip_stream) {
  return guarded([&] { as(handle)->exportState(dst, st(hip_stream)); });
}
int duck_import_state(void *handle, const void *src, void *hip_stream) {
  return guarded([&] { as(handle)->importState(src, st(hip_stream)); });
}
static void checkTask(BatchBase *b, const DuckTask *t) {
  require(t != nullptr, "null task");
  require(t->kind == DUCK_TASK_STANDING || t->kind == DUCK_TASK_LOCOMOTION ||
              t->kind == DUCK_TASK_ROLLOUT,
          "Invalid task kind");
  require(int(b->host.joints.size()) <= DUCK_MAX_JOINTS, "too many joints for a task");
  require(std::isfinite(t->control_dt) && t->control_dt > 0 && std::isfinite(t->gait_period) &&
              t->gait_period > 0 && std::isfinite(t->action_scale) && t->action_scale > 0,
          "Invalid control configuration");
  require(t->kind == DUCK_TASK_STANDING || (std::isfinite(t->tracking_sigma) && t->tracking_sigma > 0),
          "tracking sigma must be positive");
  require(b->host.bodies.size() >= 2, "task needs a root body (body 1)");
  if (t->gait)
    require(t->gait_table != nullptr && t->gait_phases >= 1, "gait: table required");
  if (t->foot_clearance || t->load_transfer) {
    const int nb = int(b->host.bodies.size());
    require(t->feet[0] >= 0 && t->feet[0] < nb && t->feet[1] >= 0 && t->feet[1] < nb,
            "gait shaping: foot body out of range");
  }
  if (t->foot_clearance)
    require(t->foot_point != nullptr && t->foot_points >= 1, "foot clearance: points required");
  if (t->load_transfer)
    require(std::isfinite(t->weight) && t->weight > 0, "load transfer: weight must be positive");
}
int duck_task_obs_dim(const DuckTask *task, int joints) {
  if (!task || joints < 0 || joints > DUCK_MAX_JOINTS)
    return -1;
  return taskObsDim(*task, joints);
}
int duck_task_targets(void *handle, const DuckTask *task, const void *actions,
                      const void *reference, const long long *episode, const void *commands,
                      void *clamped, void *target, void *hip_stream) {
  return guarded([&] {
    auto *b = as(handle);
    checkTask(b, task);
    require(reference || !task->gait || (episode && commands),
            "task targets: the gait reference needs the episode counters and commands");
    b->taskTargets(*task, actions, reference, episode, commands, clamped, target,
                   st(hip_stream));
  });
}
int duck_task_step(void *handle, const DuckTask *task, const void *action, void *last_action,
                   const void *commands, long long *episode, void *filtered, float *returns,
                   float *obs, float *reward, unsigned char *failed, unsigned char *timeout,
                   unsigned char *done, void *diag, void *hip_stream) {
  return guarded([&] {
    auto *b = as(handle);
    checkTask(b, task);
    require(action && last_action && episode && returns && obs && reward && failed && timeout &&
                done,
            "task step: null buffer");
    require(task->kind == DUCK_TASK_STANDING || commands, "task step: commands required");
    require(!(task->kind == DUCK_TASK_LOCOMOTION && task->velocity_filter) || filtered,
            "task step: filtered velocity required");
    TaskBuffers io{nullptr, const_cast<void *>(action), last_action, commands, episode,
                   filtered, returns, nullptr, obs, reward, failed, timeout, done, diag};
    b->task(*task, kTaskStep, io, st(hip_stream));
  });
}
int duck_task_reset_inputs(void *handle, const DuckTask *task, const unsigned char *reset_mask,
                           const void *joint_draws, const void *root_draws,
                           const long long *selected, int direction, double command_speed,
                           const void *commands, void *q, void *roots, void *commands_out,
                           void *hip_stream) {
  return guarded([&] {
    auto *b = as(handle);
    checkTask(b, task);
    require(q && roots, "task reset inputs: null buffer");
    require(direction < 4, "task reset inputs: direction outside the table");
    require(!(selected || direction >= 0) || (reset_mask && commands && commands_out),
            "task reset inputs: a command draw needs the reset mask and both command buffers");
    require(std::isfinite(command_speed), "task reset inputs: command speed not finite");
    b->taskResetInputs(*task, reset_mask, joint_draws, root_draws, selected, direction,
                       command_speed, commands, q, roots, commands_out, st(hip_stream));
  });
}
int duck_task_observe(void *handle, const DuckTask *task, const unsigned char *reset_mask,
                      void *actions, const void *commands, long long *episode, void *filtered,
                      float *returns, void *forces, float *obs, void *hip_stream) {
  return guarded([&] {
    auto *b = as(handle);
    checkTask(b, task);
    require(actions && episode && returns && obs, "task observe: null buffer");
    require(task->kind != DUCK_TASK_LOCOMOTION || commands, "task observe: commands required");
    require(!(task->kind == DUCK_TASK_LOCOMOTION && task->velocity_filter) || filtered,
            "task observe: filtered velocity required");
    TaskBuffers io{reset_mask, actions, actions, commands, episode, filtered, returns,
                   forces, obs, nullptr, nullptr, nullptr, nullptr, nullptr};
    b->task(*task, kTaskReset, io, st(hip_stream));
  });
}
int duck_servo(void *handle, const DuckServo *servo, const void *target, void *history,
               int cursor, unsigned char *initialized, const void *root_offset,
               void *previous_motor, void *previous_applied, void *motor, void *supply,
               void *hip_stream) {
  return guarded([&] {
    auto *b = as(handle);
    require(servo != nullptr, "null servo parameters");
    require(target && history && initialized && root_offset && previous_motor &&
                previous_applied && motor,
            "servo: null buffer");
    require(servo->lag >= 0 && servo->lag < 1024 && cursor >= 0 && cursor <= servo->lag,
            "servo: invalid lag or cursor");
    const double values[] = {servo->kt, servo->resistance, servo->dtheta_stribeck, servo->alpha,
                             servo->vin, servo->vin_min, servo->kp_fw, servo->force_limit};
    for (double v : values)
      require(std::isfinite(v), "servo: non-finite parameter");
    require(servo->resistance != 0 && servo->dtheta_stribeck != 0 && servo->vin_min > 0,
            "servo: resistance, dtheta_stribeck and vin_min must be nonzero");
    ServoBuffers io{target, history, cursor, initialized, root_offset, previous_motor,
                    previous_applied, motor, supply};
    b->servo(*servo, io, st(hip_stream));
  });
}
int duck_servo_substep(void *handle, const DuckServo *servo, const DuckServoSubstep *io,
                       void *hip_stream) {
  return guarded([&] {
    auto *b = as(handle);
    require(servo != nullptr && io != nullptr, "null servo parameters");
    require(io->target && io->history && io->initialized && io->root_offset &&
                io->previous_motor && io->previous_applied,
            "servo: null buffer");
    require(servo->lag >= 0 && servo->lag < 1024 && io->cursor >= 0 && io->cursor <= servo->lag,
            "servo: invalid lag or cursor");
    const double values[] = {servo->kt, servo->resistance, servo->dtheta_stribeck, servo->alpha,
                             servo->vin, servo->vin_min, servo->kp_fw, servo->force_limit};
    for (double v : values)
      require(std::isfinite(v), "servo: non-finite parameter");
    require(servo->resistance != 0 && servo->dtheta_stribeck != 0 && servo->vin_min > 0,
            "servo: resistance, dtheta_stribeck and vin_min must be nonzero");
    b->servoSubstep(*servo, *io, st(hip_stream));
  });
}
int duck_reference(void *handle, const void *target, const void *force, int substeps, double kp,
                   double limit, void *bodies, void *joints, void *diag) {
  return guarded(
      [&] { as(handle)->reference(target, force, substeps, kp, limit, bodies, joints, diag); });
}
int duck_reference_noalloc(void *handle, const void *target, const void *force, int substeps,
                           double kp, double limit, void *bodies, void *joints, void *diag) {
  return guarded([&] {
    as(handle)->referenceNoAlloc(target, force, substeps, kp, limit, bodies, joints, diag);
  });
}
}
