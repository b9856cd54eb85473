"""ctypes access to the CPU oracle (test infrastructure only).

`Oracle` wraps liboracle.so, this repository's restatement of the reference
AVBD step, and `OracleBatch` its threaded batch driver (the reference's
CpuBatch32/64).  `ReferenceProbe` wraps oracle/_ref/ref_probe.so, the reference's
own src/cuda/kernel.cuh compiled in place by oracle/Makefile (present only
where the reference tree was available at build time).  Both expose the same
single-environment API so the tests can check one against the other.

Only tests/, bench.py's cpu_baseline leg and smoke() may use this module.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
PROBE_LIB = HERE / "_ref" / "ref_probe.so"
REF_DIR = HERE / "_ref"

IMPLICIT_COLOURED = 0
EXPLICIT_SEQUENTIAL = 1

_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)


def _d(a):
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a, a.ctypes.data_as(_dp)


def _load(path, prefix):
    lib = ctypes.CDLL(str(path))
    sig = {
        "last_error": (ctypes.c_char_p, []),
        "destroy": (None, [ctypes.c_void_p]),
        "dims": (ctypes.c_int, [ctypes.c_void_p, _ip, _ip]),
        "reset": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp]),
        "set_controls": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp, ctypes.c_double, ctypes.c_double]),
        "set_motor": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp]),
        "advance": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
        "detect": (ctypes.c_int, [ctypes.c_void_p]),
        "failed": (ctypes.c_int, [ctypes.c_void_p]),
        "snapshot": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp, _dp]),
        "set_body": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _dp, _dp, _dp, _dp]),
        "contacts": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _ip, _ip, _dp]),
        "colors": (ctypes.c_int, [ctypes.c_void_p, _ip, _ip]),
        "joint_state": (ctypes.c_int, [ctypes.c_void_p, _dp]),
        "contact_forces": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _dp]),
        "self_contact_stats": (ctypes.c_int, [ctypes.c_void_p, _dp]),
        "contact_counts": (ctypes.c_int, [ctypes.c_void_p, _dp]),
        "generalized_loads": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, f"{prefix}_{name}")
        fn.restype = res
        fn.argtypes = args
    return lib


_libs = {}


def _lib(kind):
    if kind not in _libs:
        if kind == "oracle":
            if not ORACLE_LIB.exists():
                raise FileNotFoundError(f"{ORACLE_LIB} is not built (make -C oracle oracle)")
            lib = _load(ORACLE_LIB, "oracle")
            lib.oracle_create.restype = ctypes.c_void_p
            lib.oracle_create.argtypes = [ctypes.c_char_p, ctypes.c_double, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int]
            for name in ("set_friction", "set_mass_scale"):
                fn = getattr(lib, f"oracle_{name}")
                fn.restype = ctypes.c_int
                fn.argtypes = [ctypes.c_void_p, ctypes.c_double]
            lib.oracle_set_root_velocity.restype = ctypes.c_int
            lib.oracle_set_root_velocity.argtypes = [ctypes.c_void_p, _dp, _dp]
            lib.oracle_convex_query.restype = ctypes.c_int
            lib.oracle_convex_query.argtypes = [_dp, ctypes.c_int, _dp, ctypes.c_int, _dp,
                                                ctypes.c_double, ctypes.c_double, ctypes.c_int,
                                                _dp]
            lib.oracle_flops.restype = ctypes.c_longlong
        else:
            if not PROBE_LIB.exists():
                raise FileNotFoundError(f"{PROBE_LIB} is not built (make -C oracle ref)")
            lib = _load(PROBE_LIB, "probe")
            lib.probe_create.restype = ctypes.c_void_p
            lib.probe_create.argtypes = [ctypes.c_char_p, ctypes.c_double, ctypes.c_int,
                                         ctypes.c_int]
        _libs[kind] = lib
    return _libs[kind]


def probe_available():
    return PROBE_LIB.exists()


class _Single:
    """One environment; all arrays float64 in and out."""

    prefix = ""

    def _call(self, name, *args):
        rc = getattr(self._lib, f"{self.prefix}_{name}")(self._h, *args)
        if rc:
            err = getattr(self._lib, f"{self.prefix}_last_error")().decode()
            raise RuntimeError(err)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            getattr(self._lib, f"{self.prefix}_destroy")(h)
            self._h = None

    def _init_dims(self):
        b, j = ctypes.c_int(), ctypes.c_int()
        getattr(self._lib, f"{self.prefix}_dims")(self._h, ctypes.byref(b), ctypes.byref(j))
        self.bodies, self.joints = b.value, j.value

    def reset(self, q, root=None):
        q, qp = _d(q)
        r, rp = _d(np.zeros(6) if root is None else root)
        self._call("reset", qp, rp)

    def set_controls(self, target, force=None, kp=0.0, limit=0.0):
        t, tp = _d(target)
        f, fp = _d(np.zeros(3) if force is None else force)
        self._call("set_controls", tp, fp, float(kp), float(limit))

    def set_motor(self, motor, force=None):
        m, mp = _d(motor)
        f, fp = _d(np.zeros(3) if force is None else force)
        self._call("set_motor", mp, fp)

    def advance(self, substeps=1):
        self._call("advance", int(substeps))

    def step(self, target, force=None, substeps=1, kp=0.0, limit=0.0):
        """Controls + advance, as one CudaBatch.step of one env."""
        self.set_controls(target, force, kp, limit)
        if not self.failed:
            self.advance(substeps)

    def detect(self):
        self._call("detect")

    @property
    def failed(self):
        return bool(getattr(self._lib, f"{self.prefix}_failed")(self._h))

    def snapshot(self):
        b = np.zeros((self.bodies, 13))
        j = np.zeros((self.joints, 2))
        d = np.zeros(6)
        self._call("snapshot", b.ctypes.data_as(_dp), j.ctypes.data_as(_dp), d.ctypes.data_as(_dp))
        return b, j, d

    def set_body(self, i, x, q, v=(0, 0, 0), w=(0, 0, 0)):
        arrays = [_d(a) for a in (x, q, v, w)]
        self._call("set_body", int(i), *[p for _, p in arrays])

    def contacts(self, capacity=256):
        n = ctypes.c_int()
        ints = np.zeros((capacity, 6), dtype=np.int32)
        reals = np.zeros((capacity, 26))
        self._call("contacts", capacity, ctypes.byref(n), ints.ctypes.data_as(_ip),
                   reals.ctypes.data_as(_dp))
        return ints[: n.value].copy(), reals[: n.value].copy()

    def colors(self):
        c = np.zeros(self.bodies, dtype=np.int32)
        n = ctypes.c_int()
        self._call("colors", c.ctypes.data_as(_ip), ctypes.byref(n))
        return c, n.value

    def joint_state(self):
        out = np.zeros((self.joints, 31))
        self._call("joint_state", out.ctypes.data_as(_dp))
        return out

    def contact_forces(self, ground_only=False):
        out = np.zeros((self.bodies, 3))
        self._call("contact_forces", int(bool(ground_only)), out.ctypes.data_as(_dp))
        return out

    def self_contact_stats(self):
        out = np.zeros(2)
        self._call("self_contact_stats", out.ctypes.data_as(_dp))
        return out

    def contact_counts(self):
        out = np.zeros(2)
        self._call("contact_counts", out.ctypes.data_as(_dp))
        return out

    def generalized_loads(self, offset=(0, 0, 0)):
        o, op = _d(offset)
        out = np.zeros((self.joints, 3))
        self._call("generalized_loads", op, out.ctypes.data_as(_dp))
        return out


class Oracle(_Single):
    """This repository's restatement (mode 0 implicit-coloured, 1 explicit-sequential)."""

    prefix = "oracle"

    def __init__(self, model, dt=0.005, iterations=10, fp64=False, mode=IMPLICIT_COLOURED):
        self._lib = _lib("oracle")
        self._h = self._lib.oracle_create(str(model).encode(), float(dt), int(iterations),
                                          int(bool(fp64)), int(mode))
        if not self._h:
            raise ValueError(self._lib.oracle_last_error().decode())
        self.fp64, self.mode = bool(fp64), mode
        self._init_dims()

    def set_friction(self, mu):
        self._call("set_friction", float(mu))

    def set_mass_scale(self, s):
        self._call("set_mass_scale", float(s))

    def set_root_velocity(self, v, w=(0, 0, 0)):
        (_, vp), (_, wp) = _d(v), _d(w)
        self._call("set_root_velocity", vp, wp)


class OracleBatch:
    """The reference's CPU batch (src/cuda/cpu_bindings.cpp:20-168, CpuBatch32
    and CpuBatch64) over this restatement: `n` environments sharing one model,
    stepped by `threads` std::thread workers (environment e on worker
    e mod workers), with the same parameter checks (ValueError) and failure
    rules.  Arrays are float64 in and out."""

    _sig = {
        "create": (ctypes.c_void_p, [ctypes.c_char_p, ctypes.c_int, ctypes.c_double, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int]),
        "destroy": (None, [ctypes.c_void_p]),
        "dims": (ctypes.c_int, [ctypes.c_void_p, _ip, _ip, _ip]),
        "reset": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_ubyte), _dp, _dp]),
        "step": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp, ctypes.c_int, ctypes.c_double,
                                ctypes.c_double]),
        "step_motor": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp]),
        "state": (ctypes.c_int, [ctypes.c_void_p, _dp, _dp, _dp]),
        "contact_counts": (ctypes.c_int, [ctypes.c_void_p, _dp]),
    }

    def __init__(self, model, num_envs, dt=0.005, iterations=10, threads=1, fp64=False):
        self._lib = _lib("oracle")
        for name, (res, args) in self._sig.items():
            fn = getattr(self._lib, f"oracle_batch_{name}")
            fn.restype, fn.argtypes = res, args
        self._h = self._lib.oracle_batch_create(str(model).encode(), int(num_envs), float(dt),
                                                int(iterations), int(bool(fp64)), int(threads))
        if not self._h:
            raise ValueError(self._lib.oracle_last_error().decode())
        n, b, j = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        self._lib.oracle_batch_dims(self._h, ctypes.byref(n), ctypes.byref(b), ctypes.byref(j))
        self.num_envs, self.bodies, self.joints = n.value, b.value, j.value
        self.fp64 = bool(fp64)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.oracle_batch_destroy(h)
            self._h = None

    def _call(self, name, *args):
        if getattr(self._lib, f"oracle_batch_{name}")(self._h, *args):
            raise ValueError(self._lib.oracle_last_error().decode())

    def _shaped(self, a, shape):
        a = np.ascontiguousarray(a, dtype=np.float64)
        if a.shape != tuple(shape):
            raise ValueError("Invalid array shape")
        return a, a.ctypes.data_as(_dp)

    def reset(self, mask, q, root):
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        if m.shape != (self.num_envs,):
            raise ValueError("Invalid array shape")
        q, qp = self._shaped(q, (self.num_envs, self.joints))
        r, rp = self._shaped(root, (self.num_envs, 6))
        self._call("reset", m.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)), qp, rp)

    def step(self, target, forces, substeps, kp, limit):
        t, tp = self._shaped(target, (self.num_envs, self.joints))
        f, fp = self._shaped(forces, (self.num_envs, 3))
        self._call("step", tp, fp, int(substeps), float(kp), float(limit))

    def step_motor(self, motor, forces):
        m, mp = self._shaped(motor, (self.num_envs, self.joints, 3))
        f, fp = self._shaped(forces, (self.num_envs, 3))
        self._call("step_motor", mp, fp)

    def state(self):
        b = np.zeros((self.num_envs, self.bodies, 13))
        j = np.zeros((self.num_envs, self.joints, 2))
        d = np.zeros((self.num_envs, 6))
        self._call("state", b.ctypes.data_as(_dp), j.ctypes.data_as(_dp), d.ctypes.data_as(_dp))
        return b, j, d

    def contact_counts(self):
        out = np.zeros((self.num_envs, 2))
        self._call("contact_counts", out.ctypes.data_as(_dp))
        return out


class ReferenceProbe(_Single):
    """The reference's own kernel.cuh core, compiled in place (oracle/_ref)."""

    prefix = "probe"

    def __init__(self, model, dt=0.005, iterations=10, fp64=False):
        self._lib = _lib("probe")
        self._h = self._lib.probe_create(str(model).encode(), float(dt), int(iterations),
                                         int(bool(fp64)))
        if not self._h:
            raise ValueError(self._lib.probe_last_error().decode())
        self.fp64 = bool(fp64)
        self._init_dims()


def convex_query(va, vb, poses, inflation=0.0, tolerance=None, fp64=True):
    """Stand-alone MPR: dict(status, depth, normal, position)."""
    lib = _lib("oracle")
    if tolerance is None:
        tolerance = 1e-8 if fp64 else 1e-6
    (a, ap), (b, bp), (p, pp) = _d(va), _d(vb), _d(poses)
    out = np.zeros(8)
    rc = lib.oracle_convex_query(ap, len(a), bp, len(b), pp, float(inflation), float(tolerance),
                                 int(bool(fp64)), out.ctypes.data_as(_dp))
    if rc:
        raise ValueError(lib.oracle_last_error().decode())
    return dict(status=int(out[0]), depth=out[1], normal=out[2:5].copy(),
                position=out[5:8].copy())


def flops():
    return int(_lib("oracle").oracle_flops())


def build():
    """Compile liboracle.so (and oracle/_ref when the reference tree exists)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)
    ref = os.environ.get("DUCK_REFERENCE_ROOT", "/root/reference")
    if Path(ref).is_dir():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REF={ref}"], check=True)
