// gfx950 kernels of the batched AVBD environment step.
#pragma once
#include "../../include/duck_hip.h"
#include "avbd_step.hpp"

namespace duckhip {

// Lane (i + N) mod 16 of the same 16-lane row (DPP row_ror:N).
template <int N> __device__ __forceinline__ int rowRor(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x120 + N, 0xF, 0xF, true);
}
template <int N> __device__ __forceinline__ float rowRor(float v) {
  return __int_as_float(rowRor<N>(__float_as_int(v)));
}
template <int N> __device__ __forceinline__ double rowRor(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const unsigned lo = rowRor<N>(int(unsigned(b))), hi = rowRor<N>(int(unsigned(b >> 32)));
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Maximum over the L lanes of an environment, on every one of them.  For
// L == 16 (one DPP row) four row rotations replace the LDS-crossbar shuffles.
// c ? a : b on copies: a conditional on two lvalues of a struct type selects
// between their addresses, which keeps the object they belong to in memory.
template <class T> __device__ __forceinline__ T pickValue(bool c, T a, T b) { return c ? a : b; }

// The value of lane ^ 1 (DPP quad_perm [1, 0, 3, 2]).
__device__ __forceinline__ float laneSwap1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ double laneSwap1(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_mov_dpp(int(b), 0xB1, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp(int(b >> 32), 0xB1, 0xF, 0xF, false);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

template <class T> __device__ __forceinline__ T swizzle16(T v);
template <> __device__ __forceinline__ int swizzle16(int v) {
  return __builtin_amdgcn_ds_swizzle(v, 0x401F); // lane ^ 16 within 32-lane groups
}
template <> __device__ __forceinline__ float swizzle16(float v) {
  return __int_as_float(swizzle16(__float_as_int(v)));
}
template <> __device__ __forceinline__ double swizzle16(double v) {
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
  const unsigned lo = swizzle16(int(unsigned(b))), hi = swizzle16(int(unsigned(b >> 32)));
  return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

template <int L, class T> __device__ __forceinline__ T groupMax(T v) {
  if constexpr (L == 16 || L == 32) {
    T u = rowRor<8>(v);
    v = v > u ? v : u;
    u = rowRor<4>(v);
    v = v > u ? v : u;
    u = rowRor<2>(v);
    v = v > u ? v : u;
    u = rowRor<1>(v);
    v = v > u ? v : u;
    if constexpr (L == 32) {
      u = swizzle16(v);
      v = v > u ? v : u;
    }
    return v;
  } else {
#pragma unroll
    for (int o = L / 2; o > 0; o /= 2) {
      T u = __shfl_xor(v, o, L);
      v = v > u ? v : u;
    }
    return v;
  }
}
template <int L> __device__ __forceinline__ int groupOr(int v) {
  if constexpr (L == 16 || L == 32) {
    v |= rowRor<8>(v);
    v |= rowRor<4>(v);
    v |= rowRor<2>(v);
    v |= rowRor<1>(v);
    if constexpr (L == 32)
      v |= swizzle16(v);
    return v;
  } else {
#pragma unroll
    for (int o = L / 2; o > 0; o /= 2)
      v |= __shfl_xor(v, o, L);
    return v;
  }
}
__device__ __forceinline__ int waveMaxInt(int v) {
#pragma unroll
  for (int o = 32; o > 0; o /= 2) {
    int u = __shfl_xor(v, o, 64);
    v = v > u ? v : u;
  }
  return v;
}

// Candidate point k of ground shape si in body coordinates: hull or box
// corners are stored points; a sphere offers its lowest point and a capsule
// the lowest points of its two end spheres under the body orientation q.
template <class R>
__device__ __forceinline__ V3<R> groundPoint(const DeviceModel<R> &M, const V3<R> *points, int si,
                                              int k, Q4<R> q) {
  const int type = M.stype[si];
  if (type == 1 || type == 3)
    return points[M.soffset[si] + k];
  V3<R> c{M.center[0][si], M.center[1][si], M.center[2][si]};
  V3<R> down = rotate(conj(q), V3<R>{0, 0, -M.size[0][si]});
  if (type == 0)
    return c + down;
  Q4<R> sq{M.sq[0][si], M.sq[1][si], M.sq[2][si], M.sq[3][si]};
  return (c + rotate(sq, V3<R>{0, 0, (k ? R(1) : R(-1)) * M.size[1][si]})) + down;
}


template <class S> __device__ __forceinline__ S &blobAt(unsigned char *base, long long bytes, int e) {
  return *reinterpret_cast<S *>(base + bytes * e);
}

// The dispatcher hands consecutive workgroups to the 8 XCDs in turn, and
// each XCD has its own L2.  Workgroup b runs the environments of block
// xcdBlock(b, n) instead of block b: the workgroups of one XCD take one
// contiguous run of blocks, so the rows of the per-env inputs (targets,
// forces) that neighbouring environments share come from one L2 once.  A
// bijection of [0, n), whatever the placement, so only the speed depends on it.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcdBlock(int b, int n) {
  const int q = n / kXcds, r = n % kXcds, x = b % kXcds, k = b / kXcds;
  return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

// Copy words [a, b) of one environment's blob between HBM and LDS (both
// 16-byte aligned) with the L lanes of its group: the 16-byte interior in
// dwordx4 chunks, up to `Chunks` per lane loaded before any is stored (one
// memory round trip per Chunks * L chunks), the unaligned ends as words.
// Exactly [a, b) is written.
template <int Chunks>
__device__ __forceinline__ void copyWords(unsigned *dst, const unsigned *src, int a, int b, int lane,
                                          int L) {
  if (a >= b)
    return;
  const int a4 = (a + 3) & ~3, b4 = b & ~3;
  if (a4 >= b4) {
    for (int i = a + lane; i < b; i += L)
      dst[i] = src[i];
    return;
  }
  if (lane < a4 - a)
    dst[a + lane] = src[a + lane];
  if (lane < b - b4)
    dst[b4 + lane] = src[b4 + lane];
  const uint4 *s4 = reinterpret_cast<const uint4 *>(src + a4);
  uint4 *d4 = reinterpret_cast<uint4 *>(dst + a4);
  const int n = (b4 - a4) / 4;
  for (int c = lane; c < n; c += Chunks * L) {
    // loads unconditional (index clamped to the last chunk) so that the
    // chunks stay in registers
    uint4 v[Chunks];
#pragma unroll
    for (int k = 0; k < Chunks; ++k)
      v[k] = s4[c + k * L < n ? c + k * L : n - 1];
#pragma unroll
    for (int k = 0; k < Chunks; ++k)
      if (c + k * L < n)
        d4[c + k * L] = v[k];
  }
}

// `n` 16-byte chunks from global memory straight into LDS with the 64 lanes
// of a wave (global_load_lds_dwordx4: the chunk of lane t of instruction k
// lands at chunk 64 k + t of the destination; no registers hold the data).
// Complete once the wave's vector memory count drains.
template <int N>
__device__ __forceinline__ void dmaChunks(const unsigned char *src, __attribute__((address_space(3))) unsigned char *dst,
                                          int t) {
#pragma unroll
  for (int k = 0; k < (N + 63) / 64; ++k)
    if (t + 64 * k < N)
      __builtin_amdgcn_global_load_lds(src + 16 * (t + 64 * k), dst + 1024 * k, 16, 0, 0);
}

// The blobs of a wave's environments into LDS, first round, as LDS DMA: the
// group every step reads and writes (poses through the counts) with the first
// kWarmContacts ground contacts as one range and, with `bodies`, the
// reset-only group.  Environment g of the wave is e0 + g.
constexpr int kWarmContacts = 8;
template <class S, int G, class Env>
__device__ void loadHot(Env *envs, unsigned char *states, long long blobBytes, int e0, int count, int t,
                        bool bodies) {
  constexpr int CGcap = int(sizeof(S::gc) / sizeof(S::gc[0]));
  constexpr int gcBytes = int(sizeof(decltype(S::gc[0])));
  constexpr int hot = int(hotBegin<S>()), header = int(headerBytes<S>());
  constexpr int warm = header + (kWarmContacts < CGcap ? kWarmContacts : CGcap) * gcBytes;
  constexpr int reset = int(resetBegin<S>()), end = int(sizeof(S));
  static_assert(hot % 128 == 0 && warm % 16 == 0 && reset % 16 == 0 && end % 16 == 0,
                "copied groups are whole 16-byte chunks, group 1 starts on 128 bytes");
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (e0 + g >= count)
      break;
    const unsigned char *blob = states + blobBytes * (e0 + g);
    auto *lds = (__attribute__((address_space(3))) unsigned char *)(&envs[g].s);
    dmaChunks<(warm - hot) / 16>(blob + hot, lds + hot, t);
    if (bodies)
      dmaChunks<(end - reset) / 16>(blob + reset, lds + reset, t);
  }
}

// The rest of one environment's blob, once its counts are known: the
// further live contacts, for a launch that holds its controls (`held`) or
// sets motor channels (`motor`) the targets and force, and for a held launch
// the drive parameters.
template <class S>
__device__ void loadEnv(S &dst, const S *src, int lane, int L, bool held, bool motor) {
  constexpr int header = int(headerBytes<S>() / 4), hot = int(hotBegin<S>() / 4);
  constexpr int CGcap = int(sizeof(S::gc) / sizeof(S::gc[0]));
  constexpr int CScap = int(sizeof(S::sc) / sizeof(S::sc[0]));
  constexpr int gcWords = int(sizeof(decltype(S::gc[0])) / 4);
  constexpr int scStart = int(offsetof(S, sc) / 4), scWords = int(sizeof(decltype(S::sc[0])) / 4);
  constexpr int warm = header + (kWarmContacts < CGcap ? kWarmContacts : CGcap) * gcWords;
  int ngc = src->ngc, nsc = src->nsc;
  unsigned *d = reinterpret_cast<unsigned *>(&dst);
  const unsigned *s = reinterpret_cast<const unsigned *>(src);
  ngc = ngc < 0 ? 0 : (ngc > CGcap ? CGcap : ngc);
  nsc = nsc < 0 ? 0 : (nsc > CScap ? CScap : nsc);
  copyWords<4>(d, s, warm, header + ngc * gcWords, lane, L);
  copyWords<4>(d, s, scStart, scStart + nsc * scWords, lane, L);
  if (held || motor)
    copyWords<4>(d, s, int(targetBegin<S>() / 4), hot, lane, L);
  // the lead words in the diagnostics' first 32-byte sector: a launch that
  // steps the environment writes whole sectors (a partial one would make the
  // L2 read it first), and these words hold zeros, as the state was created
  for (int i = int(diagBegin<S>() / 32 * 8) + lane; i < int(diagBegin<S>() / 4); i += L)
    d[i] = 0;
  if (held)
    copyWords<4>(d, s, int(driveBegin<S>() / 4), int(driveEnd<S>() / 4), lane, L);
}

// What a step writes of the drive parameters and of the colouring.
enum DriveWrite { kWriteNoDrive = 0, kWriteDrive = 1, kWriteMotorDrive = 2 };

// LDS -> HBM after a step: from word `from` (the diagnostics, the force or
// group 1, by what the launch set) through the live ground contacts as one range,
// the live body contacts, and the drive parameters (all, the motor-written
// three, or none) and the colouring where they changed.  Mass, inertia and
// friction only change on reset.
template <class S>
__device__ void storeEnv(S *dst, const S &src, int lane, int L, int from, int driveWrite, bool colours) {
  constexpr int header = int(headerBytes<S>() / 4);
  constexpr int gcWords = int(sizeof(decltype(S::gc[0])) / 4);
  constexpr int scStart = int(offsetof(S, sc) / 4), scWords = int(sizeof(decltype(S::sc[0])) / 4);
  unsigned *d = reinterpret_cast<unsigned *>(dst);
  const unsigned *s = reinterpret_cast<const unsigned *>(&src);
  copyWords<16>(d, s, from, header + src.ngc * gcWords, lane, L);
  copyWords<4>(d, s, scStart, scStart + src.nsc * scWords, lane, L);
  if (driveWrite != kWriteNoDrive)
    copyWords<4>(d, s, int((driveWrite == kWriteDrive ? driveBegin<S>() : motorBegin<S>()) / 4),
                 int(driveEnd<S>() / 4), lane, L);
  if (colours)
    copyWords<4>(d, s, int(coloursBegin<S>() / 4), int(coloursEnd<S>() / 4), lane, L);
}

// MPR narrow phase between two shapes (convex.cuh:124-217).  The shape data
// come from the workgroup's staged copy (Frames: type, staged points or
// sphere/capsule data, interior point, radius); only point sets of more than
// kCachedPoints points are read from the model's point array.  With MQ == 2
// a query runs on two adjacent lanes (2k, 2k + 1): each evaluates the support
// point of one shape and the two exchange them, so both hold the same
// support point and run the same portal steps on the same values.
template <class R, int B, int J, int MQ> struct MprQuery {
  const Frames<R, B, J> &F;
  const DeviceModel<R> &M;
  const V3<R> *points;
  int sa, sb;
  V3<R> xa, xb;
  Q4<R> qa, qb;
  R inflation;
  bool second; // MQ == 2: this lane evaluates shape b's support
  // MQ == 2: the lane's own shape (index, flags, point count, pose and its
  // staged slots), read once per query so that a support point is register
  // work.
  int ownS = 0, ownFlags = 0, ownCount = 0;
  V3<R> ownX{}, ownPts[MQ == 2 ? kCachedPoints : 1];
  Q4<R> ownQ{};
  __device__ __forceinline__ V3<R> staged(int k, int s) const { return V3<R>{F.spt[k][0][s], F.spt[k][1][s], F.spt[k][2][s]}; }
  __device__ __forceinline__ void loadOwn() {
    if constexpr (MQ == 2) {
      ownS = second ? sb : sa;
      ownFlags = F.sflags[ownS];
      ownCount = F.scount[ownS];
      ownX = pickValue(second, xb, xa);
      ownQ = pickValue(second, qb, qa);
#pragma unroll
      for (int i = 0; i < kCachedPoints; ++i)
        ownPts[i] = staged(i, ownS);
    }
  }
  // support1 of the lane's own shape, from the registers loadOwn filled (a
  // sphere or capsule holds its centre, radius and half length, and axis in
  // slots 0, 1 and 2, as staged)
  __device__ __forceinline__ V3<R> supportOwn(V3<R> dir, R infl) const {
    V3<R> ld = rotate(conj(ownQ), dir), local;
    const int type = ownFlags >> 4;
    if (type == 0 || type == 2) {
      local = ownPts[0] + unitOrNan(ld) * ownPts[1].x;
      if (type == 2) {
        const V3<R> axis = ownPts[2];
        local = local + axis * (dot(axis, ld) >= 0 ? ownPts[1].y : -ownPts[1].y);
      }
    } else if (ownFlags & 2) {
      // the first maximum in index order, as a pairwise tree (a later point
      // wins only when strictly greater; slots past the count never do)
      R val[kCachedPoints];
      V3<R> pt[kCachedPoints];
#pragma unroll
      for (int i = 0; i < kCachedPoints; ++i) {
        val[i] = i < ownCount ? dot(ownPts[i], ld) : R(-INFINITY);
        pt[i] = ownPts[i];
      }
#pragma unroll
      for (int w = 1; w < kCachedPoints; w *= 2)
#pragma unroll
        for (int i = 0; i + w < kCachedPoints; i += 2 * w) {
          const bool later = val[i + w] > val[i];
          val[i] = later ? val[i + w] : val[i];
          pt[i] = pickValue(later, pt[i + w], pt[i]);
        }
      local = pt[0];
    } else {
      int best = -1;
      const int off = M.soffset[ownS];
      R value = R(-INFINITY);
      for (int i = 0; i < ownCount; ++i) {
        R cand = dot(points[off + i], ld);
        if (cand > value) {
          best = i;
          value = cand;
        }
      }
      local = points[off + (best < 0 ? 0 : best)];
    }
    return (ownX + rotate(ownQ, local)) + dir * infl;
  }
  __device__ __forceinline__ V3<R> support1(int s, V3<R> x, Q4<R> q, V3<R> dir, R infl) const {
    V3<R> ld = rotate(conj(q), dir), local;
    const int flags = F.sflags[s], type = flags >> 4;
    if (type == 0 || type == 2) {
      local = staged(0, s) + unitOrNan(ld) * F.spt[1][0][s];
      if (type == 2) {
        const V3<R> axis = staged(2, s);
        local = local + axis * (dot(axis, ld) >= 0 ? F.spt[1][1][s] : -F.spt[1][1][s]);
      }
    } else if (flags & 2) {
      // every staged slot loaded at once (slots past the count hold zeros
      // and are never chosen), then the first maximum in index order
      const int n = F.scount[s];
      R cand[kCachedPoints];
      int best[kCachedPoints];
#pragma unroll
      for (int i = 0; i < kCachedPoints; ++i) {
        cand[i] = i < n ? dot(staged(i, s), ld) : R(-INFINITY);
        best[i] = i;
      }
#pragma unroll
      for (int w = 1; w < kCachedPoints; w *= 2)
#pragma unroll
        for (int i = 0; i + w < kCachedPoints; i += 2 * w) {
          const bool later = cand[i + w] > cand[i];
          cand[i] = later ? cand[i + w] : cand[i];
          best[i] = later ? best[i + w] : best[i];
        }
      local = staged(best[0], s);
    } else {
      int best = -1, off = M.soffset[s], n = F.scount[s];
      R value = R(-INFINITY);
      for (int i = 0; i < n; ++i) {
        R cand = dot(points[off + i], ld);
        if (cand > value) {
          best = i;
          value = cand;
        }
      }
      local = points[off + (best < 0 ? 0 : best)];
    }
    return (x + rotate(q, local)) + dir * infl;
  }
  // A support point of the Minkowski difference: v = a - b, and s = a + b
  // (the two shapes' points enter the contact position only as their sum).
  struct SP {
    V3<R> v, s;
  };
  __device__ __forceinline__ SP support(V3<R> dir) const {
    SP p;
    V3<R> a, b;
    if constexpr (MQ == 2) {
      const V3<R> mine = supportOwn(second ? -dir : dir, inflation / R(2));
      const V3<R> other{laneSwap1(mine.x), laneSwap1(mine.y), laneSwap1(mine.z)};
      a = pickValue(second, other, mine);
      b = pickValue(second, mine, other);
    } else {
      a = support1(sa, xa, qa, dir, inflation / R(2));
      b = support1(sb, xb, qb, -dir, inflation / R(2));
    }
    p.v = a - b;
    p.s = a + b;
    return p;
  }
};

template <class R> struct MprHit {
  int status;
  V3<R> normal, position;
  R depth;
};

template <class R> DUCK_HD V3<R> closestToOrigin(V3<R> a, V3<R> b, V3<R> c) {
  V3<R> best = a;
  R dist = dot(a, a);
  V3<R> v[3] = {a, b, c};
  for (int i = 0; i < 3; ++i) {
    V3<R> start = v[i], edge = v[(i + 1) % 3] - start;
    R sq = dot(edge, edge);
    V3<R> p = start + edge * (sq > 0 ? clampv(-dot(start, edge) / sq, R(0), R(1)) : R(0));
    if (dot(p, p) < dist) {
      dist = dot(p, p);
      best = p;
    }
  }
  V3<R> ab = b - a, ac = c - a, n = cross(ab, ac);
  R nn = dot(n, n);
  if (nn > 0) {
    V3<R> p = n * (dot(n, a) / nn);
    R u = dot(cross(b - p, c - p), n) / nn;
    R w = dot(cross(c - p, a - p), n) / nn;
    if (u >= 0 && w >= 0 && u + w <= 1 && dot(p, p) < dist)
      best = p;
  }
  return best;
}

// The portal is four named points (p0 the interior point) whose updates are
// selected, never addressed: an indexed array here became scratch memory.
template <class R, class Query> __device__ __forceinline__ MprHit<R> mprContact(const Query &Qy, R tolerance) {
  using SP = typename Query::SP;
  auto pick = [](bool c, const SP &x, const SP &y) __attribute__((always_inline)) {
    return SP{c ? x.v : y.v, c ? x.s : y.s};
  };
  MprHit<R> hit{0, {0, 0, 0}, {0, 0, 0}, 0};
  SP p0, p1, p2, p3;
  const auto &F = Qy.F;
  V3<R> ia{F.sinterior[0][Qy.sa], F.sinterior[1][Qy.sa], F.sinterior[2][Qy.sa]};
  V3<R> ib{F.sinterior[0][Qy.sb], F.sinterior[1][Qy.sb], F.sinterior[2][Qy.sb]};
  {
    const V3<R> a = Qy.xa + rotate(Qy.qa, ia), b = Qy.xb + rotate(Qy.qb, ib);
    p0.v = a - b;
    p0.s = a + b;
  }
  R size = mx(R(0.001), F.sradius[Qy.sa] + F.sradius[Qy.sb]);
  R eps = tolerance * R(0.01);
  if (norm(p0.v) < eps)
    p0.v.x += eps * R(10);
  V3<R> dir = unitOrNan(-p0.v);
  p1 = Qy.support(dir);
  if (dot(p1.v, dir) <= 0)
    return hit;
  dir = cross(p0.v, p1.v);
  if (norm(dir) <= eps * size) {
    hit.status = 1;
    hit.depth = norm(p1.v);
    hit.normal = hit.depth > eps ? -unitOrNan(p1.v) : unitOrNan(p0.v);
    hit.position = divide(p1.s, R(2));
    return hit;
  }
  dir = unitOrNan(dir);
  p2 = Qy.support(dir);
  if (dot(p2.v, dir) <= 0)
    return hit;
  dir = unitOrNan(cross(p1.v - p0.v, p2.v - p0.v));
  if (dot(dir, p0.v) > 0) {
    const SP t = p1;
    p1 = p2;
    p2 = t;
    dir = -dir;
  }
  bool discovered = false;
  for (int it = 0; it < 128; ++it) {
    if (!mfinite(dir.x))
      break;
    p3 = Qy.support(dir);
    if (dot(p3.v, dir) <= 0)
      return hit;
    const bool into2 = dot(cross(p1.v, p3.v), p0.v) < -eps * size * size;
    const bool into1 = !into2 && dot(cross(p3.v, p2.v), p0.v) < -eps * size * size;
    if (!into2 && !into1) {
      discovered = true;
      break;
    }
    p2 = pick(into2, p3, p2);
    p1 = pick(into1, p3, p1);
    dir = unitOrNan(cross(p1.v - p0.v, p2.v - p0.v));
  }
  if (!discovered) {
    hit.status = -1;
    return hit;
  }
  auto portalDir = [&]() __attribute__((always_inline)) { return unitOrNan(cross(p2.v - p1.v, p3.v - p1.v)); };
  auto advanceOf = [&](const SP &v, V3<R> d) __attribute__((always_inline)) {
    return dot(v.v, d) - mx(dot(p1.v, d), mx(dot(p2.v, d), dot(p3.v, d)));
  };
  // The new support point replaces p1 (both sides positive, or both
  // negative), p3 (p1's side positive, p2's not) or p2 (p1's side negative,
  // p3's positive) -- the reference's choice of the portal face to keep.
  auto expand = [&](const SP &v) __attribute__((always_inline)) {
    const V3<R> c = cross(v.v, p0.v);
    const bool s1 = dot(p1.v, c) > 0, s2 = dot(p2.v, c) > 0, s3 = dot(p3.v, c) > 0;
    const bool to1 = s1 ? s2 : !s3, to3 = s1 && !s2, to2 = !s1 && s3;
    p1 = pick(to1, v, p1);
    p2 = pick(to2, v, p2);
    p3 = pick(to3, v, p3);
  };
  bool inside = false;
  for (int it = 0; it < 128; ++it) {
    dir = portalDir();
    if (!mfinite(dir.x))
      break;
    if (dot(dir, p1.v) >= -eps) {
      inside = true;
      break;
    }
    const SP sp = Qy.support(dir);
    if (dot(sp.v, dir) < 0 || advanceOf(sp, dir) <= tolerance)
      return hit;
    expand(sp);
  }
  if (!inside) {
    hit.status = -1;
    return hit;
  }
  for (int it = 0; it < 256; ++it) {
    dir = portalDir();
    if (!mfinite(dir.x))
      break;
    const SP sp = Qy.support(dir);
    if (advanceOf(sp, dir) <= tolerance) {
      V3<R> closest = closestToOrigin(p1.v, p2.v, p3.v);
      hit.depth = norm(closest);
      hit.normal = hit.depth > eps ? -divide(closest, hit.depth) : -dir;
      // Barycentric position on the portal (convex.cuh:105-123).
      R w0 = dot(cross(p1.v, p2.v), p3.v), w1 = dot(cross(p3.v, p2.v), p0.v),
        w2 = dot(cross(p0.v, p1.v), p3.v), w3 = dot(cross(p2.v, p1.v), p0.v);
      R sum = ((w0 + w1) + w2) + w3;
      if (!(sum > 0)) {
        w0 = 0;
        w1 = dot(cross(p2.v, p3.v), dir);
        w2 = dot(cross(p3.v, p1.v), dir);
        w3 = dot(cross(p1.v, p2.v), dir);
        sum = (w1 + w2) + w3;
      }
      if (!(sum > 0)) {
        hit.position = {R(NAN), R(NAN), R(NAN)};
      } else {
        V3<R> pos{0, 0, 0};
        pos = pos + p0.s * (w0 / (R(2) * sum));
        pos = pos + p1.s * (w1 / (R(2) * sum));
        pos = pos + p2.s * (w2 / (R(2) * sum));
        pos = pos + p3.s * (w3 / (R(2) * sum));
        hit.position = pos;
      }
      hit.status = mfinite(hit.position.x) ? 1 : -1;
      return hit;
    }
    expand(sp);
  }
  hit.status = -1;
  return hit;
}

// The fused servo substep's buffers and frame data (DuckServoSubstep of
// include/duck_hip.h in the batch dtype, the root rotation already inverted).
template <class R> struct ServoArgs {
  DuckServo p;
  int cursor;
  const R *target;
  R *history;
  unsigned char *initialized;
  const R *rootOffset;
  R *previousMotor, *previousApplied, *motor, *supply, *selfContacts, *selfPenetration;
  R rootInv[4];
  int numFeet;
  int feet[DUCK_MAX_FEET];
  R sites[DUCK_MAX_FEET][3];
  R *gravity, *angularVelocity, *linearVelocity, *originVelocity, *footForces, *sitePositions,
      *siteVelocities, *airTime, *contactTime, *meanVelocity;
  R meanAlpha;
};

// The servo substep's prologue (the motor channels of this substep into
// `ctl`) and epilogue (statistics and refresh quantities), defined with the
// actuator model in avbd_servo.hpp.
template <class R, int B, int J, int CG, int CS, int L, int JPL, class Env>
__device__ __forceinline__ void servoPrologue(const ServoArgs<R> &sv, const DeviceModel<R> &M, Env &E,
                                              int e, int lane, bool valid, int count,
                                              R (&ctl)[JPL][3]);
template <class R, int B, int J, int CG, int CS, class Env>
__device__ __forceinline__ void servoEpilogue(const ServoArgs<R> &sv, const DeviceModel<R> &M, Env &E,
                                              int e);

// Per-launch step: controls, `substeps` physics steps, write-back; with
// Servo, the controls are the motor channels of one servo substep and the
// launch ends with the substep's statistics and refresh quantities.
// The model's solve-time view (Frames), built once per batch by framesKernel
// into device memory; every workgroup of a step copies it into LDS whole (one
// round of loads instead of a round trip per field).  Thread t of T.
template <class R, int B, int J>
__device__ void stageFrames(Frames<R, B, J> &F, const DeviceModel<R> &M, int t, int T) {
  const int nb = M.nb, nj = M.nj, ns = M.ns, np = M.np;
  // The joint model.  The slots of absent hinges hold
  // a zero hinge between body 0 and itself: a lane without a hinge evaluates
  // one (slot 0 of a model without hinges), masked, and its finite values
  // keep the masked stamps zero.
  for (int j = t + nj; j < J; j += T) {
    F.a[j] = F.b[j] = F.limited[j] = 0;
    F.lo[j] = F.hi[j] = F.armature[j] = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      F.ra[k][j] = F.rb[k][j] = F.axisA[k][j] = F.axisB[k][j] = F.tangentA[k][j] = F.tangentB[k][j] = 0;
  }
  for (int i = t + 2 * nj; i < 2 * J; i += T)
    F.adj[i] = 0;
  for (int j = t; j < nj; j += T) {
    F.a[j] = M.ja[j];
    F.b[j] = M.jb[j];
    F.limited[j] = M.limited[j];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      F.ra[k][j] = M.ra[k][j];
      F.rb[k][j] = M.rb[k][j];
      F.axisA[k][j] = M.axisA[k][j];
      F.axisB[k][j] = M.axisB[k][j];
      F.tangentA[k][j] = M.tangentA[k][j];
      F.tangentB[k][j] = M.tangentB[k][j];
    }
    F.lo[j] = M.lo[j];
    F.hi[j] = M.hi[j];
    F.armature[j] = M.armature[j];
  }
  for (int i = t; i <= nb; i += T)
    F.adjStart[i] = M.adjStart[i];
  for (int i = t; i < 2 * nj; i += T)
    F.adj[i] = M.adjPacked[i];
  for (int i = t; i < ns; i += T)
    F.shapeFriction[i] = M.sfriction[i];
  for (int i = t; i < nb; i += T) {
    F.order[i] = M.order[i];
    F.mass[i] = M.mass[i];
  }
  for (int i = t; i < ns; i += T) {
    F.sbody[i] = M.sbody[i];
    F.sflags[i] = M.sflags[i] | M.stype[i] << 4;
    F.scount[i] = M.scount[i];
    F.sradius[i] = M.radius[i];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      F.sinterior[k][i] = M.interior[k][i];
  }
  for (int i = t; i < np; i += T)
    F.pair[i] = M.pa[i] | M.pb[i] << 8;
  for (int i = t; i < kCachedPoints * 3 * ns; i += T) {
    const int si = i % ns, c = (i / ns) % 3, k = i / (3 * ns);
    const int type = M.stype[si];
    R v = M.spts[k][c][si];
    if (type == 0 || type == 2) {
      // the shape formula's data, in the operations the narrow phase used
      // to evaluate on each support query
      const Q4<R> sq{M.sq[0][si], M.sq[1][si], M.sq[2][si], M.sq[3][si]};
      v = k == 0   ? M.center[c][si]
          : k == 1 ? (c < 2 ? M.size[c][si] : R(0))
          : k == 2 ? comp(rotate(sq, V3<R>{0, 0, 1}), c)
                   : R(0);
    }
    F.spt[k][c][si] = v;
  }
  if (t < 3)
    F.colorStart[t] = M.colorStart[t];
}

template <class R, int B, int J>
__global__ void framesKernel(const DeviceModel<R> *model, Frames<R, B, J> *out) {
  stageFrames<R, B, J>(*out, *model, threadIdx.x, blockDim.x);
}

template <class R, int B, int J, int CG, int CS, int L, int PL, bool Servo, bool Pairs>
__device__ __forceinline__ void stepBody(const StepArgs &args, const ServoArgs<R> &sv) {
  constexpr int G = 64 / L;
  // Lanes per body-pair query, pairs per round and rounds (pairs <= CS).
  constexpr int MQ = sizeof(R) == sizeof(float) && 2 * CS <= L ? 2 : 1;
  constexpr int PR = L / MQ;
  constexpr int PPL = (CS + PR - 1) / PR;
  constexpr int SPL = (B + L - 1) / L;  // shapes per lane (shapes <= B)
  using Env = EnvLds<R, B, J, CG, CS, L>;
  using State = EnvState<R, B, J, CG, CS>;
  __shared__ Frames<R, B, J> F;
  __shared__ Env envs[G];

  const DeviceModel<R> &M = *static_cast<const DeviceModel<R> *>(args.model);
  const V3<R> *points = static_cast<const V3<R> *>(args.points);
  const int t = threadIdx.x, lane = t % L, g = t / L;
  const int e = xcdBlock(blockIdx.x, gridDim.x) * G + g;
  const bool valid = e < args.count;
  Env &E = envs[g];
  // (a model without body pairs: none of their code is compiled)
  const int nb = args.nb, nj = args.nj, ns = args.ns, np = Pairs ? args.np : 0;

  // Controls and the model's per-joint defaults, loaded first so that their
  // latency overlaps the model staging and the blob copy.
  constexpr int JPL = (J + L - 1) / L;
  R ctl[JPL][3], defs[JPL][3], fin = 0;
#pragma unroll
  for (int r = 0; r < JPL; ++r) {
    const int j = lane + r * L;
    const bool in = valid && j < nj;
    const int jc = j < nj ? j : 0;
    ctl[r][0] = ctl[r][1] = ctl[r][2] = 0;
    if (!Servo && in && args.motorMode != kHeldControls) {
      if (args.motorMode == kMotorControls) {
        const R *motor = static_cast<const R *>(args.motor) + size_t(e) * nj * 3;
        ctl[r][0] = motor[3 * j];
        ctl[r][1] = motor[3 * j + 1];
        ctl[r][2] = motor[3 * j + 2];
      } else {
        ctl[r][0] = static_cast<const R *>(args.targets)[size_t(e) * nj + j];
      }
    }
    defs[r][0] = M.torque[jc];
    defs[r][1] = M.frictionloss[jc];
    defs[r][2] = M.damping[jc];
  }
  if (!Servo && valid && lane < 3 && args.motorMode != kHeldControls)
    fin = static_cast<const R *>(args.forces)[size_t(e) * 3 + lane];

  // The model's Frames image straight into LDS (global_load_lds_dwordx4:
  // lane t's 16 bytes land at chunk t of the destination, no registers held),
  // in flight together with the controls and the blob copy below.
  {
    constexpr int FC = int(sizeof(Frames<R, B, J>) / 16);
    static_assert(sizeof(Frames<R, B, J>) % 16 == 0, "the Frames image is whole dwordx4 chunks");
    const uint4 *src = static_cast<const uint4 *>(args.frames);
    auto *dst = (__attribute__((address_space(3))) uint4 *)(&F);
#pragma unroll
    for (int k = 0; k < (FC + 63) / 64; ++k)
      if (t + 64 * k < FC)
        __builtin_amdgcn_global_load_lds(src + t + 64 * k, dst + 64 * k, 16, 0, 0);
  }

  State *gs = valid ? &blobAt<State>(args.states, args.blobBytes, e) : nullptr;
  static_assert(L >= 4, "blob copies give each of the first three lanes an end word");
  static_assert(CS <= B, "the staged pair table holds B pairs");
  loadHot<State, G>(envs, args.states, args.blobBytes, e - g, args.count, t, args.bodies != 0);
  if (valid) {
    loadEnv<State>(E.s, gs, lane, L, args.motorMode == kHeldControls, args.motorMode == kMotorControls);
    if (!args.bodies) {
      // the model's masses, inertia and shape friction, as reset writes them
      for (int b = lane; b < B; b += L) {
        E.s.mass[b] = b < nb ? M.mass[b] : R(0);
#pragma unroll
        for (int k = 0; k < 3; ++k)
          E.s.inertia[k][b] = b < nb ? M.inertia[k][b] : R(0);
      }
      if (lane == 0)
        E.s.friction = R(-1);
    }
  }
  // every load of this wave, the Frames image's included, has landed
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // The staged default schedule applies to this env while no body-body
  // contact recolours it and its dynamic bodies are the model's.
  int massPattern = 0;
  if (valid)
    for (int b = lane; b < nb; b += L)
      massPattern |= (E.s.mass[b] > 0) != (F.mass[b] > 0);
  const bool defaultSchedule = groupOr<L>(massPattern) == 0;
  if constexpr (Servo)
    servoPrologue<R, B, J, CG, CS, L>(sv, M, E, e, lane, valid, args.count, ctl);

  // ---- controls (extension.cu:87-110 / kernel.cuh:448-466) ----
  int bad = 0;
  if (valid && args.motorMode != kHeldControls) {
#pragma unroll
    for (int r = 0; r < JPL; ++r) {
      if (lane + r * L >= nj)
        continue;
      if (args.motorMode == kMotorControls) {
        if (!mfinite(ctl[r][0]) || !mfinite(ctl[r][1]) || !mfinite(ctl[r][2]) || ctl[r][1] < 0 ||
            ctl[r][2] < 0)
          bad = 1;
      } else if (!mfinite(ctl[r][0])) {
        bad = 1;
      }
    }
    if (lane < 3 && !mfinite(fin))
      bad = 1;
  }
  bad = groupOr<L>(bad);
  __syncthreads();
  bool active = false;
  // What the blob's drive parameters and colouring hold before this launch
  // (read before any lane rewrites the stamps).
  int driveWrite = kWriteNoDrive;
  int writeFrom = int(hotBegin<State>() / 4);
  const int driveIn = valid ? E.s.drive : kDriveOther;
  const bool modelColoursIn = valid && E.s.modelColours != 0;
  if (valid) {
    if (args.motorMode == kHeldControls) {
      // State::advance (kernel.cuh:421-443): the controls in the state as
      // they stand
      active = !E.s.failed;
    } else if (args.motorMode == kMotorControls) {
      // setMotor applies the channels even when they are invalid (slots
      // past the last hinge hold zeros, as the state was created).
#pragma unroll
      for (int r = 0; r < JPL; ++r) {
        const int j = lane + r * L;
        if (j >= J)
          continue;
        const bool in = j < nj;
        E.s.kp[j] = 0;
        E.s.maxTorque[j] = 0;
        E.s.torque[j] = in ? ctl[r][0] : R(0);
        E.s.frictionloss[j] = in ? ctl[r][1] : R(0);
        E.s.damping[j] = in ? ctl[r][2] : R(0);
      }
      if (lane < 3)
        E.s.force[lane] = fin;
      if (lane == 0) {
        if (bad)
          E.s.failed = 1;
        E.s.drive = kDriveMotor;
      }
      driveWrite = driveIn == kDriveMotor ? kWriteMotorDrive : kWriteDrive;
      writeFrom = int(forceBegin<State>() / 32 * 8);
      active = !E.s.failed && !bad;
    } else if (!E.s.failed && !bad) {
      const R kp = R(args.kp), limit = R(args.limit);
      const bool same = driveIn == kDriveTarget && sameBits(E.s.driveKp, kp) && sameBits(E.s.driveLimit, limit);
#pragma unroll
      for (int r = 0; r < JPL; ++r) {
        const int j = lane + r * L;
        if (j >= J)
          continue;
        // slots past the last hinge hold zeros, as the state was created
        const bool in = j < nj;
        E.s.target[j] = in ? ctl[r][0] : R(0);
        E.s.kp[j] = in ? kp : R(0);
        E.s.maxTorque[j] = in ? limit : R(0);
        E.s.torque[j] = in ? defs[r][0] : R(0);
        E.s.frictionloss[j] = in ? defs[r][1] : R(0);
        E.s.damping[j] = in ? defs[r][2] : R(0);
      }
      if (lane < 3)
        E.s.force[lane] = fin;
      if (lane == 0) {
        E.s.drive = kDriveTarget;
        E.s.driveKp = kp;
        E.s.driveLimit = limit;
      }
      driveWrite = same ? kWriteNoDrive : kWriteDrive;
      active = true;
    } else if (lane == 0) {
      // invalid controls: the environment keeps its last controls and
      // colouring, which stay in the blob as they are
      E.s.failed = 1;
    }
  }
  const bool ran = active;
  // an environment that steps rewrites its diagnostics (and its targets and
  // force, set or read above)
  if (ran)
    writeFrom = int(diagBegin<State>() / 32 * 8);
  // the write-back's plan waits in LDS, not in registers across the solve
  if (valid && lane == 0)
    E.writeback = (modelColoursIn ? 1 : 0) | driveWrite << 1 | writeFrom << 8;
  if (ran && lane == 0) {
    // the step's diagnostics start afresh (slots 6 and 7 unused, zero)
    for (int k = 0; k < 8; ++k) {
      E.stepDiag[k] = 0;
      E.s.diag[k] = k == kConverged ? R(1) : R(0);
    }
  }
  __syncthreads();

  Stepper<R, B, J, CG, CS, L, PL, Pairs> stp{M, points, F, E, lane};
  // Block-solve lanes: with P == 2, lanes l and l ^ 8 (same 16-lane DPP row)
  // share a body; `slot` numbers the bodies a colour pass runs at once.
  constexpr int P = Stepper<R, B, J, CG, CS, L, PL, Pairs>::P;
  static_assert(P == 1 || L % (8 * P) == 0, "split block solves need 8 P-lane groups");
  const int part = (lane >> 3) & (P - 1);
  const int slot = P == 1 ? lane : (lane & 7) + 8 * (lane / (8 * P));
  const R h = M.dt, alpha = M.alpha, gamma = M.gamma, ag = alpha * gamma;

  for (int sub = 0; sub < args.substeps; ++sub) {
    if (!__any(active))
      break;
    // ---------------- detection: body-body pairs (kernel.cuh:656-722) ----
    // (before the ground manifolds, so that the narrow phase does not hold
    // the ground passes' warm-start registers)
    struct PairGeom {
      V3<R> n, t1, t2, local, localB;
      R c0, lambda[3], penalty[3];
      int src;
    };
    PairGeom pg[PPL];
#pragma unroll
    for (int r = 0; r < PPL; ++r) {
      // the lanes of a query compute the same values and branch alike; the
      // first of them records the outcome
      const int pi = lane / MQ + r * PR;
      const bool lead = lane % MQ == 0;
      if (!active || pi >= np)
        continue;
      if (lead)
        E.pairHit[pi] = 0;
      const int sa = F.pair[pi] & 255, sb = F.pair[pi] >> 8, A = F.sbody[sa], Bb = F.sbody[sb];
      if (E.s.mass[A] == 0 && E.s.mass[Bb] == 0)
        continue;
      V3<R> xa = stp.X(A), xb = stp.X(Bb);
      Q4<R> qa = stp.Q(A), qb = stp.Q(Bb);
      R skin = R(.003) + h * (norm(stp.Vel(A) - stp.Vel(Bb)) + norm(stp.Omega(A)) * F.sradius[sa] +
                              norm(stp.Omega(Bb)) * F.sradius[sb]);
      if (norm(xa - xb) > F.sradius[sa] + F.sradius[sb] + skin)
        continue;
      MprQuery<R, B, J, MQ> qy{F, M, points, sa, sb, xa, xb, qa, qb, skin, lane % MQ == 1};
      qy.loadOwn();
      MprHit<R> hit = mprContact(qy, mx(R(1e-8), M.tolerance * R(.1)));
      if (hit.status < 0) {
        E.s.failed = 1;
        continue;
      }
      if (hit.status == 0)
        continue;
      PairGeom &o = pg[r];
      o.n = hit.normal;
      o.t1 = unitOrNan(cross(mabs(o.n.x) < R(.8) ? V3<R>{1, 0, 0} : V3<R>{0, 1, 0}, o.n));
      o.t2 = cross(o.n, o.t1);
      R gap = skin - hit.depth;
      o.local = rotate(conj(qa), (hit.position + o.n * (gap / R(2))) - xa);
      o.localB = rotate(conj(qb), (hit.position - o.n * (gap / R(2))) - xb);
      o.c0 = mn(gap, R(0));
      o.src = -1;
      for (int i = 0; i < E.s.nsc; ++i) {
        const SelfContact<R> &old = E.s.sc[i];
        V3<R> on{old.n[0], old.n[1], old.n[2]};
        V3<R> ol{old.local[0], old.local[1], old.local[2]},
            olb{old.localB[0], old.localB[1], old.localB[2]};
        if (scShape(old.id) == sa && scOtherShape(old.id) == sb && dot(on, o.n) > R(.95) &&
            norm(rotate(qa, ol - o.local)) < R(.005) && norm(rotate(qb, olb - o.localB)) < R(.005)) {
          o.src = i;
          break;
        }
      }
      if (o.src >= 0) {
        // the source's force in the new basis, read while the previous list
        // is still in LDS
        const SelfContact<R> &old = E.s.sc[o.src];
        V3<R> f = ((V3<R>{old.t1[0], old.t1[1], old.t1[2]} * old.lambda[0]) +
                   (V3<R>{old.t2[0], old.t2[1], old.t2[2]} * old.lambda[1])) +
                  (V3<R>{old.n[0], old.n[1], old.n[2]} * old.lambda[2]);
        o.lambda[0] = dot(f, o.t1);
        o.lambda[1] = dot(f, o.t2);
        o.lambda[2] = dot(f, o.n);
        for (int d = 0; d < 3; ++d)
          o.penalty[d] = old.penalty[d];
      }
      if (lead)
        E.pairHit[pi] = 1;
    }
    // ---------------- detection: ground manifolds (kernel.cuh:601-653) ----
    // Per pick: point index | (warm-start source + 1) << 20, so that only
    // four registers per shape live across the barrier into compaction.
    int picks[SPL][4], npick[SPL];
    struct WarmGround {
      R lambda[3], penalty[3], local[3], anchor[2];
      bool stick;
    };
    WarmGround warm[SPL][4];
#pragma unroll
    for (int r = 0; r < SPL; ++r) {
      npick[r] = 0;
#pragma unroll
      for (int p = 0; p < 4; ++p)
        picks[r][p] = 0;
      const int si = lane + r * L;
      if (!active || si >= ns)
        continue;
      const int b = F.sbody[si], flags = F.sflags[si];
      const R mass = E.s.mass[b];
      if (!(flags & 1) || mass == 0) {
        E.shapeCount[si] = 0;
        continue;
      }
      V3<R> x = stp.X(b), v = stp.Vel(b), w = stp.Omega(b);
      Q4<R> q = stp.Q(b);
      const R gz = M.gravity[2] + stp.forceZ(b) / mass;
      R low = mn(x.z, x.z + h * v.z + h * h * gz);
      if (double(low - F.sradius[si] * (R(1) + h * norm(w))) >= .003) {
        E.shapeCount[si] = 0;
        continue;
      }
      const int count = F.scount[si];
      const bool staged = (flags & 2) != 0;
      V3<R> chosen[4];
      int n = 0;
      if (count <= kCachedPoints) {
        // Predicted heights and world xy of every point, evaluated once as
        // one straight-line block; entries past `count` come from zero
        // points and never enter the candidate mask.
        R wz[kCachedPoints], wx[kCachedPoints], wy[kCachedPoints];
        // body-frame points: staged in LDS, or formed from the shape (a
        // branch, so that staged shapes never evaluate the shape formula)
        V3<R> pts[kCachedPoints];
        if (staged) {
#pragma unroll
          for (int k = 0; k < kCachedPoints; ++k)
            pts[k] = V3<R>{F.spt[k][0][si], F.spt[k][1][si], F.spt[k][2][si]};
        } else {
#pragma unroll
          for (int k = 0; k < kCachedPoints; ++k)
            pts[k] = k < count ? groundPoint(M, points, si, k, q) : V3<R>{0, 0, 0};
        }
#pragma unroll
        for (int k = 0; k < kCachedPoints; ++k) {
          V3<R> world = x + rotate(q, pts[k]);
          V3<R> vel = v + cross(w, world - x);
          wz[k] = mn(world.z, world.z + h * vel.z + h * h * gz);
          wx[k] = world.x;
          wy[k] = world.y;
        }
        // Pass pk of the reference takes the lowest (height, index) among the
        // points below 3 mm that are not within 5 mm (xy) of a chosen point.
        // Equivalently, candidates are visited in ascending (height, index)
        // order and each is kept unless it lies within 5 mm of a kept one: a
        // dropped candidate stays dropped (the kept set only grows), so each
        // round consumes one candidate, found by a pairwise-tree minimum.
        unsigned avail = 0;
#pragma unroll
        for (int k = 0; k < kCachedPoints; ++k)
          avail |= (k < count && double(wz[k]) < .003) ? 1u << k : 0u;
        R keptX[3] = {0, 0, 0}, keptY[3] = {0, 0, 0};
        for (int t = 0; t < kCachedPoints; ++t) {
          if (avail == 0 || n == 4)
            break;
          R tz[kCachedPoints], tx[kCachedPoints], ty[kCachedPoints];
          int tk[kCachedPoints];
#pragma unroll
          for (int k = 0; k < kCachedPoints; ++k) {
            tz[k] = ((avail >> k) & 1u) ? wz[k] : R(INFINITY);
            tx[k] = wx[k];
            ty[k] = wy[k];
            tk[k] = k;
          }
          // the left operand holds the lower indices: equal heights keep it
#pragma unroll
          for (int st = 1; st < kCachedPoints; st <<= 1)
#pragma unroll
            for (int k = 0; k < kCachedPoints; k += 2 * st) {
              const bool right = tz[k + st] < tz[k];
              tz[k] = right ? tz[k + st] : tz[k];
              tx[k] = right ? tx[k + st] : tx[k];
              ty[k] = right ? ty[k + st] : ty[k];
              tk[k] = right ? tk[k + st] : tk[k];
            }
          avail &= ~(1u << tk[0]);
          bool dup = false;
#pragma unroll
          for (int cc = 0; cc < 3; ++cc)
            dup = dup | ((cc < n) & withinFiveMm(keptX[cc] - tx[0], keptY[cc] - ty[0]));
          if (!dup) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
              picks[r][cc] = cc == n ? tk[0] : picks[r][cc];
              if (cc < 3) {
                keptX[cc] = cc == n ? tx[0] : keptX[cc];
                keptY[cc] = cc == n ? ty[0] : keptY[cc];
              }
            }
            ++n;
          }
        }
      } else {
#pragma unroll
        for (int pk = 0; pk < 4; ++pk) {
          if (n < pk)
            break;
          int best = -1;
          R lowest = R(INFINITY);
          V3<R> bestWorld{0, 0, 0};
          for (int k = 0; k < count; ++k) {
            V3<R> local = groundPoint(M, points, si, k, q), world = x + rotate(q, local);
            V3<R> vel = v + cross(w, world - x);
            R z = mn(world.z, world.z + h * vel.z + h * h * gz);
            if (double(z) >= .003 || z >= lowest)
              continue;
            bool dup = false;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
              if (cc < pk && withinFiveMm(chosen[cc].x - world.x, chosen[cc].y - world.y))
                dup = true;
            if (dup)
              continue;
            best = k;
            lowest = z;
            bestWorld = world;
          }
          if (best >= 0) {
            picks[r][pk] = best;
            chosen[pk] = bestWorld;
            n = pk + 1;
          }
        }
      }
      npick[r] = n;
      E.shapeCount[si] = n;
      // Warm-start source in the previous list (still in LDS): the first
      // entry with this shape and feature.  One pass from the end of the
      // list, four independent loads per round, the last match kept; ids
      // are compared on their shape and feature fields (`key` is -1 for an
      // absent pick, which no masked id equals).
      int src[4] = {0, 0, 0, 0}, key[4];
#pragma unroll
      for (int p = 0; p < 4; ++p)
        key[p] = p < n ? gcPack(si, 0, picks[r][p], false) : -1;
      const int ngc = E.s.ngc;
      for (int i0 = (ngc - 1) & ~3; i0 >= 0; i0 -= 4) {
        int ids[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          ids[j] = E.s.gc[i0 + j < ngc ? i0 + j : 0].id;
#pragma unroll
        for (int j = 3; j >= 0; --j) {
          const int masked = i0 + j < ngc ? ids[j] & kGcShapeFeature : -2;
#pragma unroll
          for (int p = 0; p < 4; ++p)
            src[p] = masked == key[p] ? i0 + j + 1 : src[p];
        }
      }
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        if (p < n)
          picks[r][p] |= src[p] << 20;
        // the source's multipliers, penalties and stick anchor, read while
        // the previous list is still in LDS (compaction overwrites it)
        const GroundContact<R> &old = E.s.gc[p < n && src[p] > 0 ? src[p] - 1 : 0];
        WarmGround &wm = warm[r][p];
#pragma unroll
        for (int d = 0; d < 3; ++d) {
          wm.lambda[d] = old.lambda[d];
          wm.penalty[d] = old.penalty[d];
          wm.local[d] = old.local[d];
        }
        wm.anchor[0] = old.anchor[0];
        wm.anchor[1] = old.anchor[1];
        wm.stick = gcStick(old.id);
      }
    }
    __syncthreads();
    // ---------------- compaction + warm start ----------------------------
    if (active) {
      int total = 0;
      for (int si = 0; si < ns; ++si)
        total += E.shapeCount[si];
      if (total > CG && lane == 0)
        E.s.failed = 1;
#pragma unroll
      for (int r = 0; r < SPL; ++r) {
        const int si = lane + r * L;
        if (si >= ns || npick[r] == 0)
          continue;
        int offset = 0;
        for (int k = 0; k < si; ++k)
          offset += E.shapeCount[k];
        const int b = F.sbody[si];
        V3<R> x = stp.X(b);
        Q4<R> q = stp.Q(b);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          if (p >= npick[r] || offset + p >= CG)
            break;
          GroundContact<R> c;
          const int feature = picks[r][p] & 0xFFFFF, src = (picks[r][p] >> 20) - 1;
          V3<R> local;
          if (F.sflags[si] & 2)
            local = V3<R>{F.spt[feature][0][si], F.spt[feature][1][si], F.spt[feature][2][si]};
          else
            local = groundPoint(M, points, si, feature, q);
          const V3<R> world = x + rotate(q, local);
          R lam[3] = {0, 0, 0}, pen[3] = {1000, 1000, 1000};
          R anchor[2] = {world.x, world.y};
          if (src >= 0) {
            const WarmGround &old = warm[r][p];
            for (int d = 0; d < 3; ++d) {
              lam[d] = old.lambda[d];
              pen[d] = old.penalty[d];
            }
            if (old.stick) {
              local = {old.local[0], old.local[1], old.local[2]};
              anchor[0] = old.anchor[0];
              anchor[1] = old.anchor[1];
            }
          }
          c.id = gcPack(si, b, feature, false);
          c.local[0] = local.x;
          c.local[1] = local.y;
          c.local[2] = local.z;
          c.anchor[0] = anchor[0];
          c.anchor[1] = anchor[1];
          c.c0 = mn((x + rotate(q, local)).z, R(0));
          for (int d = 0; d < 3; ++d) {
            c.lambda[d] = lam[d] * ag;
            c.penalty[d] = clampv(pen[d] * gamma, R(1000), R(1e9));
          }
          E.s.gc[offset + p] = c;
          clearContactPadding(E.s.gc[offset + p]);
        }
      }
      if (lane == 0)
        E.s.ngc = total > CG ? CG : total;
#pragma unroll
      for (int r = 0; r < PPL; ++r) {
        const int pi = lane / MQ + r * PR;
        if (lane % MQ != 0 || pi >= np || !E.pairHit[pi])
          continue;
        int slot = 0;
        for (int k = 0; k < pi; ++k)
          slot += E.pairHit[k];
        if (slot >= CS) {
          E.s.failed = 1;
          continue;
        }
        const PairGeom &o = pg[r];
        const int sa = F.pair[pi] & 255, sb = F.pair[pi] >> 8;
        SelfContact<R> c;
        c.id = scPack(F.sbody[sa], F.sbody[sb], sa, sb, false);
        R lam[3] = {0, 0, 0}, pen[3] = {1000, 1000, 1000};
        if (o.src >= 0) {
          for (int d = 0; d < 3; ++d) {
            lam[d] = o.lambda[d];
            pen[d] = o.penalty[d];
          }
        }
        V3<R> vs[5] = {o.local, o.localB, o.t1, o.t2, o.n};
        R *dst[5] = {c.local, c.localB, c.t1, c.t2, c.n};
        for (int v = 0; v < 5; ++v) {
          dst[v][0] = vs[v].x;
          dst[v][1] = vs[v].y;
          dst[v][2] = vs[v].z;
        }
        c.c0 = o.c0;
        c.friction = M.pfriction[pi];
        for (int d = 0; d < 3; ++d) {
          c.lambda[d] = lam[d] * ag;
          c.penalty[d] = clampv(pen[d] * gamma, R(1000), R(1e9));
        }
        E.s.sc[slot] = c;
        clearContactPadding(E.s.sc[slot]);
      }
    }
    __syncthreads();
    // ---------------- colours (kernel.cuh:596-598, 717-720) -------------
    int pairHits = 0;
    for (int pi = 0; pi < np; ++pi)
      pairHits += E.pairHit[pi];
    const bool fresh = active && !(pairHits == 0 && defaultSchedule);
    if (active) {
      for (int b = lane; b < B; b += L) {
        // slots past the last body hold zeros, as the state was created
        E.s.colors[b] = b < nb ? M.colors[b] : 0;
        if (!fresh && b < nb)
          E.order[b] = F.order[b];
      }
      if (!fresh && lane < 3)
        E.colorStart[lane] = F.colorStart[lane];
      if (lane < 8)
        E.stepDiag[lane] = 0;
      if (!fresh && lane == 0) {
        E.s.nsc = 0;
        E.s.colorCount = 2;
      }
    }
    __syncthreads();
    if (fresh && lane == 0) {
      // each body contact between bodies of one colour gives its second
      // body a new colour, in list order (later contacts see the change)
      const int nsc = pairHits < CS ? pairHits : CS;
      E.s.nsc = nsc;
      int cc = 2;
      for (int i = 0; i < nsc; ++i) {
        int a = scBody(E.s.sc[i].id), b = scOther(E.s.sc[i].id);
        if (E.s.mass[a] > 0 && E.s.mass[b] > 0 && E.s.colors[a] == E.s.colors[b])
          E.s.colors[b] = cc++;
      }
      E.s.colorCount = cc;
    }
    __syncthreads();
    // The fresh schedule: the dynamic bodies of each colour in index order,
    // placed by ballots over the environment's lanes (body b = lane + r L).
    const int freshColours = __builtin_amdgcn_readfirstlane(waveMaxInt(fresh ? E.s.colorCount : 0));
    if (freshColours > 0) {
      constexpr int BR = (B + L - 1) / L;
      const uint64_t group = (L == 64 ? ~uint64_t(0) : (uint64_t(1) << L) - 1) << (g * L);
      int col[BR];
#pragma unroll
      for (int r = 0; r < BR; ++r) {
        const int b = lane + r * L;
        col[r] = fresh && b < nb && E.s.mass[b] > 0 ? E.s.colors[b] : -1;
      }
      int start = 0;
      for (int c = 0; c <= freshColours; ++c) {
        if (fresh && lane == 0)
          E.colorStart[c] = start;
        if (c == freshColours)
          break;
#pragma unroll
        for (int r = 0; r < BR; ++r) {
          const uint64_t m = __ballot(col[r] == c) & group;
          const int below = __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0));
          if (col[r] == c)
            E.order[start + below] = lane + r * L;
          start += __popcll(m);
        }
      }
    }
    __syncthreads();
    if (active && E.s.failed)
      active = false; // detection failure ends this env's launch
    // ---------------- warm start, predictor, contact masks ---------------
    if (active) {
      for (int ji = lane; ji < nj; ji += L) {
        auto je = stp.evalJoint(ji);
#pragma unroll
        for (int k = 0; k < 7; ++k)
          E.c0[k][ji] = je.C[k];
        E.angle0[ji] = je.angle;
        E.s.lambdaF[ji] *= ag;
        E.s.penaltyF[ji] = clampv(E.s.penaltyF[ji] * gamma, R(1), R(1e7));
        const int a = F.a[ji], b = F.b[ji];
        E.velocity0[ji] = dot(stp.Omega(b) - stp.Omega(a), je.axis);
#pragma unroll
        for (int k = 0; k < 7; ++k) {
          E.s.lambda[k][ji] *= ag;
          E.s.penalty[k][ji] =
              clampv(E.s.penalty[k][ji] * gamma, k < 3 ? R(1000) : R(1), k < 3 ? R(1e9) : R(1e7));
        }
      }
    }
    // The per-body contact masks, cleared here and filled below by one LDS
    // atomic or per contact from the contact's lane.
    constexpr int GW = (CG + 63) / 64;
    if (active) {
      for (int b = lane; b < B; b += L) {
#pragma unroll
        for (int k = 0; k < GW; ++k)
          E.gmask[k][b] = 0;
        E.smask[b] = 0;
      }
    }
    __syncthreads(); // joint warm start reads the poses the predictor overwrites
    if (active) {
      for (int i = lane; i < E.s.ngc; i += L)
        atomicOr(reinterpret_cast<unsigned long long *>(&E.gmask[i >> 6][gcBody(E.s.gc[i].id)]),
                 1ull << (i & 63));
      for (int i = lane; i < E.s.nsc; i += L) {
        const int id = E.s.sc[i].id;
        atomicOr(&E.smask[scBody(id)], 1u << i);
        atomicOr(&E.smask[scOther(id)], 1u << i);
      }
      for (int b = lane; b < nb; b += L) {
        V3<R> x = stp.X(b);
        Q4<R> q = stp.Q(b);
#pragma unroll
        for (int k = 0; k < 3; ++k)
          E.x0[k][b] = comp(x, k);
        E.q0[0][b] = q.w;
        E.q0[1][b] = q.x;
        E.q0[2][b] = q.y;
        E.q0[3][b] = q.z;
        {
          R iw[6];
          inertiaWorld(q, stp.Inertia(b), iw);
          for (int k = 0; k < 6; ++k)
            E.Iw[k][b] = iw[k];
        }
        const R mass = E.s.mass[b];
        if (mass == 0)
          continue;
        V3<R> v = stp.Vel(b), w = stp.Omega(b), I = stp.Inertia(b);
        V3<R> xp = faxpy(h * h, V3<R>{M.gravity[0], M.gravity[1], M.gravity[2]} + divide(stp.force(b), mass),
                         faxpy(h, v, x));
        V3<R> spin = -cross(w, stp.inertiaApply(q, I, w, false));
        V3<R> wp = faxpy(h, stp.inertiaApply(q, I, spin, true), w);
        Q4<R> qp = fqmul(fexpmap(h * wp), q);
#pragma unroll
        for (int k = 0; k < 3; ++k)
          E.xp[k][b] = comp(xp, k);
        E.qp[0][b] = qp.w;
        E.qp[1][b] = qp.x;
        E.qp[2][b] = qp.y;
        E.qp[3][b] = qp.z;
        stp.setX(b, xp);
        stp.setQ(b, qp);
      }
    }
    int colours = waveMaxInt(active ? E.s.colorCount : 0);
    __syncthreads();
    // When each of the first two colours fits in one pass of the block-solve
    // slots, every lane's body for them is fixed for the whole step.
    bool twoColourSlots = false;
    int mine[2] = {-1, -1}, partOf[2] = {part, part}, partsOf[2] = {P, P};
    if (active) {
      const int c0 = E.colorStart[0], c1 = E.colorStart[1], c2 = E.colorStart[2];
      twoColourSlots = c1 - c0 <= L / P && c2 - c1 <= L / P;
      if (c0 + slot < c1)
        mine[0] = E.order[c0 + slot];
      if (c1 + slot < c2)
        mine[1] = E.order[c1 + slot];
    }
    // A third colour that holds one body (a body contact recoloured it) whose
    // hinges all end at colour-0 or static bodies: none of its rows but the
    // body contacts reads a pose that the colour-1 pass moves, so the free
    // slot of colour 1 assembles them during that pass (bit 28 of its plan's
    // first word), and the third pass adds the body-contact rows and solves.
    // The sums and their order are those of one assembly in the third pass,
    // unless a lane of the wave leaves the fast forms in one of the two passes
    // and not the other (the generic assembly orders a body's rows otherwise;
    // float only, within rounding).
    bool early = false, stageLane = false;
    if constexpr (sizeof(R) == sizeof(float) && P == 2 && Pairs) {
      if (active && twoColourSlots && E.s.colorCount == 3) {
        const int c1 = E.colorStart[1], c2 = E.colorStart[2];
        if (E.colorStart[3] - c2 == 1 && c2 - c1 < L / P) {
          const int b3 = E.order[c2];
          bool ok = true;
          for (int a = F.adjStart[b3]; a < F.adjStart[b3 + 1]; ++a) {
            const int packed = F.adj[a], ja = (packed >> 8) & 255, jb = (packed >> 16) & 255;
            const int other = ja == b3 ? jb : ja;
            ok = ok && (E.s.mass[other] <= 0 || E.s.colors[other] == 0);
          }
          early = ok;
          stageLane = ok && slot == c2 - c1;
          if (stageLane)
            mine[1] = b3;
          if (ok && lane == 0) {
            E.earlyMask = E.smask[b3];
            E.smask[b3] = 0;
          }
        }
      }
    }
    if constexpr (P == 2) {
      // A colour with a free slot lends it to the body that four lanes
      // serve best (the most assembly rounds saved, weighed below); that
      // body's group becomes four lanes (both slots, lane and lane ^ 8).
      if (active && twoColourSlots) {
        // Each slot weighs its own body, and one reduction over the
        // environment's lanes picks the first of the heaviest (the lanes of
        // an environment are active together).
        int bestOf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int cs = E.colorStart[c], n = E.colorStart[c + 1] - cs;
          int key = 0;
          if (slot < n && n < L / P && !(c == 1 && early)) {
            // What four lanes save over two: the hinge rounds (ceil(h / 2)
            // against ceil(h / 4)) and the contact rounds beyond the two
            // straight-line ones per lane, a hinge's rows costing about
            // three contacts' (instruction counts of the float assembly).
            const int b = E.order[cs + slot];
            const int hinges = F.adjStart[b + 1] - F.adjStart[b];
            const int ground = stp.groundCount(b);
            const int hingeRounds = ((hinges + 1) >> 1) - ((hinges + 3) >> 2);
            const int extra2 = ((ground + 1) >> 1) - 2, extra4 = ((ground + 3) >> 2) - 2;
            const int contactRounds = (extra2 > 0 ? extra2 : 0) - (extra4 > 0 ? extra4 : 0);
            const int saved = 3 * hingeRounds + contactRounds;
            key = saved > 0 ? (saved << 8 | (255 - slot)) : 0;
          }
          key = groupMax<L>(key);
          bestOf[c] = key != 0 ? 255 - (key & 255) : -1;
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int cs = E.colorStart[c], n = E.colorStart[c + 1] - cs;
          const int best = bestOf[c];
          if (best < 0)
            continue;
          // The busy body takes slots 0 and 4 (order within a colour is free:
          // same-colour bodies do not interact), so that one DPP row
          // rotation by 12 meets the two slots' pair sums in both; the bodies
          // it displaces move to the slot it left and to the free slot 7.
          const int busy = E.order[cs + best];
          if (slot == 0) {
            mine[c] = busy;
            partsOf[c] = 4;
          } else if (slot == 4) {
            mine[c] = busy;
            partOf[c] = part + 2;
            partsOf[c] = 4;
          } else if (slot == best) {
            mine[c] = E.order[cs]; // best is neither 0 nor 4 here
          } else if (slot == 7) {
            // displaced from slot 4 (or from slot 0 when the busy body was at 4)
            mine[c] = best == 4 ? E.order[cs] : (n > 4 ? E.order[cs + 4] : -1);
          }
        }
      }
    }
    // The lane's assembly plans for its bodies of the first two colours.
    typename Stepper<R, B, J, CG, CS, L, PL, Pairs>::SlotPlan plans[2] = {{0, 0}, {0, 0}};
    if constexpr (sizeof(R) == sizeof(float)) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
        if (active && twoColourSlots && mine[c] >= 0)
          plans[c] = stp.plan(mine[c], partOf[c], partsOf[c]);
      plans[1].w0 |= stageLane ? 1 << 28 : 0;
    }
    E.early = early ? 1 : 0;
    // Which hinge's dual update a lane makes first.  A hinge's dual update
    // and the next iteration's first-colour block solve of its colour-0 body
    // evaluate it at the same poses (nothing moves in between), so when every
    // environment of the wave has fixed first-colour slots, each lane updates
    // the hinge its first-colour slot stamps first and that slot reuses the
    // evaluation.  Hinges no such slot stamps (`leftover`) go round-robin.
    const bool shareEval = sizeof(R) == sizeof(float) && P == 2 && __all(!active || twoColourSlots);
    const uint32_t allJoints = nj >= 32 ? ~0u : (1u << nj) - 1;
    int dualJoint = lane < nj ? lane : -1;
    uint32_t leftover = L >= 32 ? 0u : allJoints & ~((1u << (L & 31)) - 1);
    if (shareEval) {
      dualJoint = active && mine[0] >= 0 && ((plans[0].w0 >> 24) & 1) ? plans[0].w0 & 255 : -1;
      leftover = allJoints & ~uint32_t(groupOr<L>(dualJoint >= 0 ? int(1u << dualJoint) : 0));
      if constexpr (L == 16) {
        // The lanes left without a hinge take the leftover ones (the n-th
        // such lane of the environment the n-th leftover hinge), so that
        // the straight-line block updates them too; only hinges beyond the
        // free lanes go round-robin.  A hinge's update does not depend on
        // the lane that makes it.
        const uint32_t freeLanes = uint32_t(__ballot(dualJoint < 0) >> (t - lane)) & 0xffffu;
        const int rank = __popc(freeLanes & ((1u << lane) - 1));
        uint32_t m = leftover;
#pragma unroll
        for (int k = 0; k < L - 1; ++k)
          m = k < rank ? m & (m - 1) : m;
        const int take = dualJoint < 0 && m != 0 ? __builtin_ctz(m) : -1;
        leftover &= ~uint32_t(groupOr<L>(take >= 0 ? int(1u << take) : 0));
        dualJoint = take >= 0 ? take : dualJoint;
      }
    }
    // The ends of that hinge and the owner of the lane's first ground
    // contact (the list is fixed until the next detection).
    const int ends0 = dualJoint >= 0 ? F.a[dualJoint] | F.b[dualJoint] << 8 : F.a[0] | F.b[0] << 8;
    typename Stepper<R, B, J, CG, CS, L, PL, Pairs>::JointEval lastEval{};
    int owner0 = 0;
    if (active && lane < E.s.ngc) {
      const int id = E.s.gc[lane].id;
      owner0 = gcBody(id) | gcShape(id) << 8;
    }
    // Contact rounds of the dual update for the whole wave (scalars; the
    // lists are fixed until the next detection).
    const int groundRounds = __builtin_amdgcn_readfirstlane(waveMaxInt(active ? E.s.ngc : 0));
    const int selfRounds = Pairs ? __builtin_amdgcn_readfirstlane(waveMaxInt(active ? E.s.nsc : 0)) : 0;
    // ---------------- AVBD iterations (kernel.cuh:979-1063) ---------------
    bool dualRan = false;
    R dJoint = 0, dAxis = 0, dDepth = 0;
    // Convergence is decided from group maxima, identical in every lane of
    // an environment, so each lane keeps the flag in a register.
    bool converged = false;
    // Whether a colour pass has a four-lane group anywhere in the wave (a
    // lane that stops iterating keeps its group's combine an identity).
    const bool quadPass0 = P == 2 && __any(active && twoColourSlots && partsOf[0] == 4);
    const bool quadPass1 = P == 2 && __any(active && twoColourSlots && partsOf[1] == 4);
    for (int it = 0; it < M.iterations; ++it) {
      const bool work = active && !converged;
      if (!__any(work))
        break;
      R maxUpdate = 0;
      for (int c = 0; c < colours; ++c) {
        const bool quadPass = c == 0 ? quadPass0 : (c == 1 ? quadPass1 : false);
        if (work && c < E.s.colorCount) {
          if (c < 2 && twoColourSlots) {
            const bool c0 = c == 0;
            const int bi = c0 ? mine[0] : mine[1];
            const bool reuse = c0 && shareEval && dualRan;
            if (bi >= 0 && reuse)
              maxUpdate = mx(maxUpdate, stp.template updateBody<true>(bi, true, partOf[0], partsOf[0],
                                                                      quadPass, plans[0], &lastEval));
            else if (bi >= 0)
              maxUpdate = mx(maxUpdate, stp.updateBody(bi, true, c0 ? partOf[0] : partOf[1],
                                                       c0 ? partsOf[0] : partsOf[1], quadPass,
                                                       c0 ? plans[0] : plans[1]));
          } else {
            // (an early-assembled third colour is its one body: slot 0)
            for (int k = E.colorStart[c] + slot; k < E.colorStart[c + 1]; k += L / P) {
              const int bi = E.order[k];
              maxUpdate = mx(maxUpdate, stp.updateBody(bi, true, part, P, false, stp.plan(bi, part, P),
                                                       nullptr, c == 2 && E.early != 0));
            }
          }
        }
        __syncthreads();
      }
      maxUpdate = groupMax<L>(maxUpdate);
      R error = 0;
      if (work) {
        // The lane's first hinge and first ground contact as one straight-
        // line block (stores at its end), then any further ones; the error
        // is folded in the reference's order (hinges, then contacts).  The
        // constraint values of the last iteration's dual update are the
        // step's diagnostics (the poses do not move after it).
        const int ngc = E.s.ngc;
        R errC0 = 0;
        dualRan = true;
        dJoint = dAxis = dDepth = 0;
        auto foldJoint = [&](const typename Stepper<R, B, J, CG, CS, L, PL, Pairs>::JointDual &jd) {
#pragma unroll
          for (int k = 0; k < 3; ++k)
            dJoint = mx(dJoint, mabs(jd.C[k]));
#pragma unroll
          for (int k = 3; k < 5; ++k)
            dAxis = mx(dAxis, mabs(jd.C[k]));
        };
        static_assert(L <= CG, "a lane's first contact slot exists");
        // a lane without a hinge evaluates an existing slot and stores nothing
        const bool hasJoint = dualJoint >= 0;
        // New force, penalties and stick flag of body contact i (kernel.cuh:
        // 1029-1052), stored when v; returns its depth and its term of the
        // error (folded by the caller).
        const int nsc = E.s.nsc;
        auto selfDual = [&](int i, bool v) __attribute__((always_inline)) {
          SelfContact<R> &c = E.s.sc[v ? i : 0];
          V3<R> ra, rb;
          V3<R> C = stp.selfC(c, ra, rb);
          const R depth = mx(R(0), -(C.z + alpha * c.c0));
          V3<R> f = contactForce(C, c.lambda, c.penalty, c.friction);
          R trial = fhypot(fmad(c.penalty[0], C.x, c.lambda[0]), fmad(c.penalty[1], C.y, c.lambda[1]));
          bool stick = trial <= -c.friction * f.z && double(fhypot(C.x, C.y)) < 1e-5;
          R fk[3] = {f.x, f.y, f.z}, Ck[3] = {C.x, C.y, C.z};
          if (v) {
            c.id = (c.id & 0x7fffffff) | (stick ? int(0x80000000u) : 0);
#pragma unroll
            for (int k = 0; k < 3; ++k) {
              c.lambda[k] = fk[k];
              if (f.z < 0 && (k == 2 || trial <= -c.friction * f.z))
                c.penalty[k] = mn(fmad(M.betaLinear, mabs(Ck[k]), c.penalty[k]), R(1e9));
            }
          }
          return V3<R>{depth, mx(R(0), -C.z), R(0)};
        };
        auto j0 = stp.jointDual(hasJoint ? dualJoint : (lane < J ? lane : 0), hasJoint, error, ends0);
        const auto g0 = stp.groundDual(lane, lane < ngc, errC0, owner0);
        // with body pairs, the lane's first body contact in the same block
        // (its terms are folded after the ground contacts', as the rounds do);
        // not in the fused servo substep, where it measured 2 % slower
        constexpr bool selfInBlock = Pairs && !Servo;
        V3<R> s0{0, 0, 0};
        if constexpr (selfInBlock)
          s0 = selfDual(lane, lane < nsc);
        if (__any(j0.wide) && j0.wide)
          error = stp.frictionDual(j0, wrapAngle(j0.angle));
        lastEval = j0.je;
        // unconditional: a lane past the last contact rewrites its unused
        // slot with the values it holds
        stp.storeGroundDual(lane, g0);
        if (hasJoint) {
          stp.storeJointDual(dualJoint, j0);
          foldJoint(j0);
        }
        int nth = 0;
        for (uint32_t m = leftover; m; m &= m - 1, ++nth) {
          if (nth % L != lane)
            continue;
          const int ji = __builtin_ctz(m);
          auto jd = stp.jointDual(ji, true, error, F.a[ji] | F.b[ji] << 8);
          if (jd.wide)
            error = stp.frictionDual(jd, wrapAngle(jd.angle));
          stp.storeJointDual(ji, jd);
          foldJoint(jd);
        }
        if (lane < ngc) {
          error = mx(error, errC0);
          dDepth = mx(dDepth, g0.depth);
        }
        // Further ground contacts and the body contacts run in rounds counted
        // for the whole wave (scalar trip counts, predicated bodies): a loop
        // that lanes leave at different trips ends in a block entered with
        // exec zero, and this compiler has placed the copy of a loop-carried
        // maximum there, before exec is restored, losing it.  A lane with no
        // contact in a round rewrites its own first slot with its values.
        for (int i0 = L; i0 < groundRounds; i0 += L) {
          const int i = i0 + lane;
          const bool v = i < ngc;
          const int k = v ? i : lane;
          const int id = E.s.gc[k].id;
          const auto gd = stp.groundDual(k, v, error, v ? gcBody(id) | gcShape(id) << 8 : owner0);
          stp.storeGroundDual(k, gd);
          dDepth = v ? mx(dDepth, gd.depth) : dDepth;
        }
        if constexpr (selfInBlock) {
          const bool v = lane < nsc;
          dDepth = v ? mx(dDepth, s0.x) : dDepth;
          error = v ? mx(error, s0.y) : error;
        }
        for (int i0 = selfInBlock ? L : 0; i0 < selfRounds; i0 += L) {
          const int i = i0 + lane;
          const bool v = i < nsc;
          const V3<R> sd = selfDual(i, v);
          dDepth = v ? mx(dDepth, sd.x) : dDepth;
          error = v ? mx(error, sd.y) : error;
        }
      }
      error = groupMax<L>(error);
      const bool conv = maxUpdate < M.tolerance && error < M.tolerance;
      if (work && lane == 0) {
        E.stepDiag[kIterations] = R(it + 1);
        E.stepDiag[kConverged] = conv ? R(1) : R(0);
      }
      converged = converged || (work && conv);
      __syncthreads();
    }
    // ---------------- velocity recovery (kernel.cuh:1064-1073) ------------
    if (active) {
      const R invh = R(1) / h;
      for (int b = lane; b < nb; b += L) {
        if (E.s.mass[b] == 0)
          continue;
        V3<R> x = stp.X(b), x0{E.x0[0][b], E.x0[1][b], E.x0[2][b]};
        V3<R> v = (x - x0) * invh;
        V3<R> w = flogmap(fqmul(stp.Q(b), conj(stp.Q0(b)))) * invh;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          E.s.v[k][b] = comp(v, k);
          E.s.w[k][b] = comp(w, k);
        }
        if (!mfinite(norm(x) + norm(v) + norm(w)))
          E.s.failed = 1;
      }
    }
    __syncthreads();
    if (active && E.s.failed)
      active = false;
    // ---------------- diagnostics and substep summary ---------------------
    R jointErr = dJoint, axisErr = dAxis, pen = dDepth;
    if (active && !dualRan) {
      for (int ji = lane; ji < nj; ji += L) {
        auto je = stp.evalJoint(ji);
#pragma unroll
        for (int k = 0; k < 3; ++k)
          jointErr = mx(jointErr, mabs(je.C[k]));
#pragma unroll
        for (int k = 3; k < 5; ++k)
          axisErr = mx(axisErr, mabs(je.C[k]));
      }
      for (int i = lane; i < E.s.ngc; i += L) {
        V3<R> ra;
        V3<R> C = stp.groundC(E.s.gc[i], ra);
        pen = mx(pen, mx(R(0), -(C.z + alpha * E.s.gc[i].c0)));
      }
      for (int i = lane; i < E.s.nsc; i += L) {
        V3<R> ra, rb;
        V3<R> C = stp.selfC(E.s.sc[i], ra, rb);
        pen = mx(pen, mx(R(0), -(C.z + alpha * E.s.sc[i].c0)));
      }
    }
    jointErr = groupMax<L>(jointErr);
    axisErr = groupMax<L>(axisErr);
    pen = groupMax<L>(pen);
    if (active && lane == 0) {
      R *d = E.s.diag;
      d[kJointError] = mx(d[kJointError], jointErr);
      d[kAxisError] = mx(d[kAxisError], axisErr);
      d[kPenetration] = mx(d[kPenetration], pen);
      d[kContacts] = mx(d[kContacts], R(E.s.ngc + E.s.nsc));
      d[kConverged] = (d[kConverged] != 0 && E.stepDiag[kConverged] != 0) ? R(1) : R(0);
      d[kIterations] += E.stepDiag[kIterations];
    }
    __syncthreads();
    __syncthreads();
  }
  if constexpr (Servo)
    if (valid && lane == 0)
      servoEpilogue<R, B, J, CG, CS>(sv, M, E, e);
  // The colouring of an environment that stepped is the model's exactly when
  // no body took a fresh colour; it is written when the blob holds another.
  const int plan = valid ? E.writeback : 0;
  const bool modelColours = E.s.colorCount == 2;
  const bool writeColours = ran && !(modelColours && (plan & 1));
  __syncthreads();
  if (ran && lane == 0)
    E.s.modelColours = modelColours ? 1 : 0;
  __syncthreads();
  if (valid)
    storeEnv<State>(gs, E.s, lane, L, plan >> 8, (plan >> 1) & 3, writeColours);
}

// Pairs false: for a model without body pairs.  The code starts on a 32 KiB
// boundary: the same instructions placed elsewhere in the code object have
// measured 1.5 % slower (the instruction cache sets their hot loops map to).
template <class R, int B, int J, int CG, int CS, int L, int PL = defaultSolveLanes(L), bool Pairs = true>
__global__ __launch_bounds__(64) __attribute__((aligned(32768))) void advanceKernel(StepArgs args) {
  const ServoArgs<R> none{};
  stepBody<R, B, J, CG, CS, L, PL, false, Pairs>(args, none);
}

// One servo substep per launch (bam_env.py:307-337 with refresh()), on a
// 32 KiB boundary like advanceKernel.
template <class R, int B, int J, int CG, int CS, int L, int PL = defaultSolveLanes(L), bool Pairs = true>
__global__ __launch_bounds__(64) __attribute__((aligned(32768))) void servoStepKernel(StepArgs args,
                                                                                   ServoArgs<R> servo) {
  stepBody<R, B, J, CG, CS, L, PL, true, Pairs>(args, servo);
}

} // namespace duckhip
