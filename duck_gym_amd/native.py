"""`CudaBatch`: the reference's native batch interface over libduck_hip.so.

Mirrors the pybind11 class of src/cuda/extension.cu:436-452 (constructor
arguments, method names, shapes, dtypes and error behaviour): inputs are
caller-owned device tensors checked exactly as extension.cu:206-213 checks
them (device, dtype, contiguity, shape -> RuntimeError), outputs are fresh
tensors, and every call is asynchronous on the current torch stream.  The
physics runs in the HIP kernels of libduck_hip.so; there is no CPU fallback:
constructing a batch without the built library raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "libduck_hip.so"
_lib = None


def library():
    """Load libduck_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(
                f"{LIBRARY} is missing: build it with `python -m duck_gym_amd.hipbuild` "
                "(the HIP extension is required; there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIBRARY))
        vp, ip, cp = ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p
        dbl = ctypes.c_double
        sig = {
            "duck_create": (ip, [cp, ip, dbl, ip, ip, ip, ctypes.c_uint, ctypes.POINTER(vp)]),
            "duck_create_text": (ip, [cp, ip, dbl, ip, ip, ip, ctypes.c_uint, ctypes.POINTER(vp)]),
            "duck_destroy": (None, [vp]),
            "duck_model_info": (ip, [cp, ctypes.c_uint, ctypes.POINTER(ip)]),
            "duck_dims": (ip, [vp, ctypes.POINTER(ip), ctypes.POINTER(ip), ctypes.POINTER(ip)]),
            "duck_num_envs": (ip, [vp]),
            "duck_fp_bits": (ip, [vp]),
            "duck_state_bytes": (ctypes.c_longlong, [vp]),
            "duck_kernel_info": (ip, [vp, ip, ctypes.POINTER(ctypes.c_longlong)]),
            "duck_sequential_step": (ip, [vp, ip, ip, ip]),
            "duck_joint_name": (cp, [vp, ip]),
            "duck_reset": (ip, [vp, vp, vp, vp, vp, vp]),
            "duck_step": (ip, [vp, vp, vp, ip, dbl, dbl, vp]),
            "duck_step_motor": (ip, [vp, vp, vp, vp]),
            "duck_advance": (ip, [vp, ip, vp]),
            "duck_state": (ip, [vp, vp, vp, vp, vp]),
            "duck_contact_forces": (ip, [vp, ip, vp, vp]),
            "duck_self_contact_stats": (ip, [vp, vp, vp]),
            "duck_contact_counts": (ip, [vp, vp, vp]),
            "duck_generalized_loads": (ip, [vp, vp, vp, vp]),
            "duck_reference": (ip, [vp, vp, vp, ip, dbl, dbl, vp, vp, vp]),
            "duck_reference_noalloc": (ip, [vp, vp, vp, ip, dbl, dbl, vp, vp, vp]),
            "duck_state_layout": (ip, [vp, ctypes.POINTER(ctypes.c_longlong)]),
            "duck_export_state": (ip, [vp, vp, vp]),
            "duck_import_state": (ip, [vp, vp, vp]),
            "duck_last_error": (cp, []),
            "duck_task_obs_dim": (ip, [ctypes.POINTER(DuckTask), ip]),
            "duck_task_targets": (ip, [vp, ctypes.POINTER(DuckTask)] + [vp] * 7),
            "duck_task_step": (ip, [vp, ctypes.POINTER(DuckTask)] + [vp] * 13),
            "duck_task_observe": (ip, [vp, ctypes.POINTER(DuckTask)] + [vp] * 9),
            "duck_task_reset_inputs": (ip, [vp, ctypes.POINTER(DuckTask), vp, vp, vp, vp, ip, dbl,
                                            vp, vp, vp, vp, vp]),
            "duck_servo": (ip, [vp, ctypes.POINTER(DuckServo), vp, vp, ip] + [vp] * 7),
            "duck_servo_substep": (ip, [vp, ctypes.POINTER(DuckServo),
                                        ctypes.POINTER(DuckServoSubstep), vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


EXPORTED = (
    "duck_create", "duck_create_text", "duck_destroy", "duck_model_info", "duck_dims", "duck_num_envs", "duck_fp_bits",
    "duck_state_bytes", "duck_kernel_info", "duck_joint_name", "duck_reset", "duck_step",
    "duck_step_motor", "duck_advance",
    "duck_state", "duck_contact_forces", "duck_self_contact_stats", "duck_contact_counts",
    "duck_generalized_loads", "duck_reference", "duck_reference_noalloc", "duck_state_layout",
    "duck_export_state",
    "duck_import_state", "duck_last_error", "duck_task_obs_dim", "duck_task_targets",
    "duck_task_step", "duck_task_observe", "duck_task_reset_inputs", "duck_servo",
    "duck_servo_substep",
    "duck_sequential_step",
)

MAX_JOINTS = 32


class DuckServo(ctypes.Structure):
    """`DuckServo` of include/duck_hip.h: XL330/m6 actuator parameters."""

    _fields_ = [(name, ctypes.c_double) for name in (
        "kt", "resistance", "dtheta_stribeck", "alpha", "friction_base", "friction_stribeck",
        "load_friction_external", "load_friction_motor", "load_friction_external_stribeck",
        "load_friction_motor_stribeck", "load_friction_external_quad",
        "load_friction_motor_quad", "friction_viscous", "vin", "vin_drop_gain", "vin_min",
        "kp_fw", "kp_scale", "kd_scale", "friction_scale", "force_limit")] + [
        ("lag", ctypes.c_int)]
MAX_FEET = 4


class DuckServoSubstep(ctypes.Structure):
    """`DuckServoSubstep` of include/duck_hip.h: buffers and frame data of
    one fused servo substep."""

    _fields_ = [
        ("target", ctypes.c_void_p), ("history", ctypes.c_void_p), ("cursor", ctypes.c_int),
        ("initialized", ctypes.c_void_p), ("root_offset", ctypes.c_void_p),
        ("previous_motor", ctypes.c_void_p), ("previous_applied", ctypes.c_void_p),
        ("motor", ctypes.c_void_p), ("supply", ctypes.c_void_p),
        ("self_contacts", ctypes.c_void_p), ("self_penetration", ctypes.c_void_p),
        ("root_principal_quat", ctypes.c_double * 4), ("num_feet", ctypes.c_int),
        ("foot_bodies", ctypes.c_int * MAX_FEET), ("foot_sites", (ctypes.c_double * 3) * MAX_FEET),
        ("gravity", ctypes.c_void_p), ("angular_velocity", ctypes.c_void_p),
        ("linear_velocity", ctypes.c_void_p), ("origin_velocity", ctypes.c_void_p),
        ("foot_forces", ctypes.c_void_p), ("site_positions", ctypes.c_void_p),
        ("site_velocities", ctypes.c_void_p), ("air_time", ctypes.c_void_p),
        ("contact_time", ctypes.c_void_p), ("mean_velocity", ctypes.c_void_p),
        ("mean_velocity_alpha", ctypes.c_double)]


TASK_STANDING, TASK_LOCOMOTION, TASK_ROLLOUT = 0, 1, 2


class DuckTask(ctypes.Structure):
    """`DuckTask` of include/duck_hip.h: the constants of one tensor-env task."""

    _fields_ = [
        ("kind", ctypes.c_int), ("velocity_filter", ctypes.c_int),
        ("home", ctypes.c_double * MAX_JOINTS), ("lower", ctypes.c_double * MAX_JOINTS),
        ("upper", ctypes.c_double * MAX_JOINTS), ("iquat", ctypes.c_double * 4),
        ("root_height", ctypes.c_double), ("action_scale", ctypes.c_double),
        ("control_dt", ctypes.c_double), ("gait_period", ctypes.c_double),
        ("tracking_weight", ctypes.c_double), ("heading_weight", ctypes.c_double),
        ("tracking_sigma", ctypes.c_double), ("velocity_alpha", ctypes.c_double),
        ("fall_height", ctypes.c_double), ("max_episode_length", ctypes.c_longlong),
        ("gait", ctypes.c_int), ("foot_clearance", ctypes.c_int),
        ("load_transfer", ctypes.c_int), ("gait_phases", ctypes.c_int),
        ("gait_table", ctypes.c_void_p), ("gait_lift", ctypes.c_double),
        ("feet", ctypes.c_int * 2), ("foot_points", ctypes.c_int),
        ("foot_point", ctypes.c_void_p), ("weight", ctypes.c_double),
    ]


def _raise(code, what):
    """Map a C-ABI error code to the exception the reference raises:
    TORCH_CHECK and std::runtime_error -> RuntimeError, std::invalid_argument
    (model.hpp) -> ValueError."""
    msg = library().duck_last_error().decode()
    if code == 2:
        raise ValueError(f"{what}: {msg}")
    if code == 3:
        raise RuntimeError(f"{what}: HIP failure: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def _flags(specialized, shared_memory, split_solve=False):
    return (1 if specialized else 0) | (2 if split_solve else 0) | (4 if shared_memory else 0)


def check_model(model, specialized=False, shared_memory=False):
    """Parse and validate a `.duck` model as CudaBatch(model, ...) does,
    without a device (duck_model_info): returns the counts, or raises the
    exception the constructor would (RuntimeError for an unreadable or
    malformed file and for the specialized layout checks, ValueError for a
    flattening or capacity violation)."""
    out = (ctypes.c_int * 6)()
    code = library().duck_model_info(str(model).encode(),
                                     _flags(specialized, shared_memory), out)
    if code:
        _raise(code, "CudaBatch")
    keys = ("bodies", "joints", "shapes", "pairs", "ground_capacity", "self_capacity")
    return dict(zip(keys, list(out)))


class CudaBatch:
    """Batched AVBD environments on one MI355X (gfx950) device."""

    def __init__(self, model, num_envs, dt=0.001, iterations=200, device=0, fp64=False,
                 specialized=False, shared_memory=False, split_solve=False):
        # `shared_memory` (with `specialized` only, as extension.cu:424
        # requires) is accepted for signature compatibility: the gfx950
        # kernel always stages environment state in LDS.  `split_solve` (an
        # extension) runs float64 batches in the float layout: two lanes per
        # body block solve, whose partial systems are summed in another order.
        self._create(library().duck_create, str(model), num_envs, dt, iterations, device, fp64,
                     _flags(specialized, shared_memory, split_solve))

    @classmethod
    def from_text(cls, text, num_envs, dt=0.001, iterations=200, device=0, fp64=False,
                  specialized=False, shared_memory=False, split_solve=False):
        """A batch of the model whose `.duck` text is `text` (no file; the
        same checks and errors as the constructor)."""
        self = cls.__new__(cls)
        self._create(library().duck_create_text, str(text), num_envs, dt, iterations, device,
                     fp64, _flags(specialized, shared_memory, split_solve))
        return self

    def _create(self, create, source, num_envs, dt, iterations, device, fp64, flags):
        lib = library()
        self._h = None
        handle = ctypes.c_void_p()
        code = create(source.encode(), int(num_envs), float(dt), int(iterations), int(device),
                      64 if fp64 else 32, flags, ctypes.byref(handle))
        if code:
            _raise(code, "CudaBatch")
        self._h = handle
        self.device = torch.device("cuda", int(device))
        self.dtype = torch.float64 if fp64 else torch.float32
        self.num_envs = int(num_envs)
        self.dt = float(dt)
        b, j, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        lib.duck_dims(self._h, ctypes.byref(b), ctypes.byref(j), ctypes.byref(c))
        self.num_bodies, self.num_joints, self.contact_capacity = b.value, j.value, c.value
        self._names = [lib.duck_joint_name(self._h, i).decode() for i in range(self.num_joints)]

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.duck_destroy(self._h)
            self._h = None

    @property
    def joint_names(self):
        return list(self._names)

    @property
    def state_bytes(self):
        return int(library().duck_state_bytes(self._h))

    def kernel_info(self, kernel="step"):
        """Resources of the kernel `step` ("step") or `servo_substep`
        ("servo_substep") launches (duck_kernel_info): VGPRs, static LDS bytes
        per workgroup, scratch bytes per lane, resident workgroups per CU,
        lanes and environments per workgroup, workgroups per launch, and the
        waves per SIMD they give."""
        which = {"step": 0, "servo_substep": 1}[kernel]
        out = (ctypes.c_longlong * 7)()
        code = library().duck_kernel_info(self._h, which, out)
        if code:
            _raise(code, "kernel_info")
        keys = ("vgprs", "lds_bytes_per_workgroup", "scratch_bytes_per_lane",
                "workgroups_per_cu", "lanes_per_workgroup", "envs_per_workgroup",
                "workgroups_per_launch")
        info = dict(zip(keys, (int(v) for v in out)))
        info["waves_per_simd"] = info["workgroups_per_cu"] * info["lanes_per_workgroup"] / 64 / 4
        return info

    # --------------------------------------------------------------- checks
    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def _check(self, t, shape, dtype=None):
        dtype = self.dtype if dtype is None else dtype
        if not (isinstance(t, torch.Tensor) and t.is_cuda and t.device.index == self.device.index
                and t.dtype == dtype and t.is_contiguous() and list(t.shape) == list(shape)):
            raise RuntimeError("Invalid CUDA tensor device/dtype/shape/contiguity")
        t.record_stream(torch.cuda.current_stream(self.device))
        return ctypes.c_void_p(t.data_ptr())

    def _empty(self, *shape):
        return torch.empty(shape, device=self.device, dtype=self.dtype)

    # ------------------------------------------------------------- methods
    def reset(self, mask, q, root, ext=None):
        E, J = self.num_envs, self.num_joints
        args = [self._check(mask, [E], torch.bool), self._check(q, [E, J]),
                self._check(root, [E, 6]),
                None if ext is None else self._check(ext, [E, 5])]
        with torch.cuda.device(self.device):
            code = library().duck_reset(self._h, *args, self._stream())
        if code:
            _raise(code, "reset")

    def step(self, target, forces, substeps, kp, limit):
        E, J = self.num_envs, self.num_joints
        t, f = self._check(target, [E, J]), self._check(forces, [E, 3])
        with torch.cuda.device(self.device):
            code = library().duck_step(self._h, t, f, int(substeps), float(kp), float(limit),
                                       self._stream())
        if code:
            _raise(code, "step")

    def step_motor(self, motor, forces):
        E, J = self.num_envs, self.num_joints
        m, f = self._check(motor, [E, J, 3]), self._check(forces, [E, 3])
        with torch.cuda.device(self.device):
            code = library().duck_step_motor(self._h, m, f, self._stream())
        if code:
            _raise(code, "step_motor")

    def advance(self, substeps=1):
        """`substeps` steps with the controls the state holds (duck_advance:
        kernel.cuh's State::advance; CudaBatch has no such method -- the
        C++ duck::Solver steps this way)."""
        with torch.cuda.device(self.device):
            code = library().duck_advance(self._h, int(substeps), self._stream())
        if code:
            _raise(code, "advance")

    def state(self):
        E = self.num_envs
        b = self._empty(E, self.num_bodies, 13)
        j = self._empty(E, self.num_joints, 2)
        d = self._empty(E, 6)
        with torch.cuda.device(self.device):
            code = library().duck_state(self._h, ctypes.c_void_p(b.data_ptr()),
                                        ctypes.c_void_p(j.data_ptr()),
                                        ctypes.c_void_p(d.data_ptr()), self._stream())
        if code:
            _raise(code, "state")
        return b, j, d

    def contact_forces(self, ground_only=False):
        out = self._empty(self.num_envs, self.num_bodies, 3)
        with torch.cuda.device(self.device):
            code = library().duck_contact_forces(self._h, int(bool(ground_only)),
                                                 ctypes.c_void_p(out.data_ptr()), self._stream())
        if code:
            _raise(code, "contact_forces")
        return out

    def self_contact_stats(self):
        out = self._empty(self.num_envs, 2)
        with torch.cuda.device(self.device):
            code = library().duck_self_contact_stats(self._h, ctypes.c_void_p(out.data_ptr()),
                                                     self._stream())
        if code:
            _raise(code, "self_contact_stats")
        return out

    def contact_counts(self):
        out = self._empty(self.num_envs, 2)
        with torch.cuda.device(self.device):
            code = library().duck_contact_counts(self._h, ctypes.c_void_p(out.data_ptr()),
                                                 self._stream())
        if code:
            _raise(code, "contact_counts")
        return out

    def generalized_loads(self, offset):
        o = self._check(offset, [self.num_envs, 3])
        out = self._empty(self.num_envs, self.num_joints, 3)
        with torch.cuda.device(self.device):
            code = library().duck_generalized_loads(self._h, o, ctypes.c_void_p(out.data_ptr()),
                                                    self._stream())
        if code:
            _raise(code, "generalized_loads")
        return out

    def reference(self, target, forces, substeps, kp, limit):
        J = self.num_joints
        if not (isinstance(target, torch.Tensor) and target.device.type == "cpu"
                and target.is_contiguous() and target.dtype == self.dtype
                and list(target.shape) == [J]):
            raise RuntimeError("Invalid CPU reference target")
        if not (isinstance(forces, torch.Tensor) and forces.device.type == "cpu"
                and forces.is_contiguous() and list(forces.shape) == [3]
                and forces.dtype == self.dtype and substeps > 0):
            raise RuntimeError("Invalid CPU reference inputs")
        b = torch.empty(self.num_bodies, 13, dtype=self.dtype)
        j = torch.empty(J, 2, dtype=self.dtype)
        d = torch.empty(6, dtype=self.dtype)
        with torch.cuda.device(self.device):
            torch.cuda.synchronize(self.device)
            code = library().duck_reference(
                self._h, ctypes.c_void_p(target.data_ptr()), ctypes.c_void_p(forces.data_ptr()),
                int(substeps), float(kp), float(limit), ctypes.c_void_p(b.data_ptr()),
                ctypes.c_void_p(j.data_ptr()), ctypes.c_void_p(d.data_ptr()))
        if code:
            _raise(code, "reference")
        return b, j, d

    # ------------------------------------------------------ servo substep
    def servo(self, params, target, history, cursor, initialized, root_offset, previous_motor,
              previous_applied, supply=None):
        """One BAM servo substep (include/duck_hip.h duck_servo); returns the
        motor channels [E,J,3] for `step_motor`."""
        E, J = self.num_envs, self.num_joints
        lag = int(params.lag)
        motor = self._empty(E, J, 3)
        args = [self._check(target, [E, J]), self._check(history, [lag + 1, E, J]),
                ctypes.c_int(int(cursor)), self._check(initialized, [E], torch.bool),
                self._check(root_offset, [E, 3]), self._check(previous_motor, [E, J]),
                self._check(previous_applied, [E, J]), ctypes.c_void_p(motor.data_ptr()),
                self._ptr(supply, [E])]
        with torch.cuda.device(self.device):
            code = library().duck_servo(self._h, ctypes.byref(params), *args, self._stream())
        if code:
            _raise(code, "servo")
        return motor

    # ---------------------------------------------- tensor-env control step
    def _ptr(self, t, shape, dtype=None):
        return None if t is None else self._check(t, shape, dtype)

    def servo_substep(self, params, target, history, cursor, initialized, root_offset,
                      previous_motor, previous_applied, *, root_principal_quat=(1.0, 0, 0, 0),
                      feet=(), foot_sites=None, motor=None, supply=None, self_contacts=None,
                      self_penetration=None, gravity=None, angular_velocity=None,
                      linear_velocity=None, origin_velocity=None, foot_forces=None,
                      site_positions=None, site_velocities=None, air_time=None,
                      contact_time=None, mean_velocity=None, mean_velocity_alpha=0.0):
        """One fused BAM substep (include/duck_hip.h duck_servo_substep): the
        servo, the motor step with zero root force, the self-contact maxima,
        the refresh() quantities and, with `mean_velocity` [E,3], the
        mean-velocity filter mean += alpha (origin velocity - mean)
        (bam_env.py:343-345), in one launch.  Outputs are written into the
        tensors given (any may be None); in/out tensors are updated in place."""
        E, J = self.num_envs, self.num_joints
        F = len(feet)
        if F > MAX_FEET:
            raise RuntimeError("servo substep: invalid foot count")
        io = DuckServoSubstep()
        io.target = self._check(target, [E, J]).value
        io.history = self._check(history, [int(params.lag) + 1, E, J]).value
        io.cursor = int(cursor)
        io.initialized = self._check(initialized, [E], torch.bool).value
        io.root_offset = self._check(root_offset, [E, 3]).value
        io.previous_motor = self._check(previous_motor, [E, J]).value
        io.previous_applied = self._check(previous_applied, [E, J]).value
        for name, t, shape in (("motor", motor, [E, J, 3]), ("supply", supply, [E]),
                               ("self_contacts", self_contacts, [E]),
                               ("self_penetration", self_penetration, [E]),
                               ("gravity", gravity, [E, 3]),
                               ("angular_velocity", angular_velocity, [E, 3]),
                               ("linear_velocity", linear_velocity, [E, 3]),
                               ("origin_velocity", origin_velocity, [E, 3]),
                               ("foot_forces", foot_forces, [E, F, 3]),
                               ("site_positions", site_positions, [E, F, 3]),
                               ("site_velocities", site_velocities, [E, F, 3]),
                               ("air_time", air_time, [E, F]), ("contact_time", contact_time, [E, F]),
                               ("mean_velocity", mean_velocity, [E, 3])):
            ptr = self._ptr(t, shape)
            setattr(io, name, None if ptr is None else ptr.value)
        io.mean_velocity_alpha = float(mean_velocity_alpha)
        for k in range(4):
            io.root_principal_quat[k] = float(root_principal_quat[k])
        io.num_feet = F
        sites = [[0.0, 0.0, 0.0]] * F if foot_sites is None else foot_sites
        for f in range(F):
            io.foot_bodies[f] = int(feet[f])
            for k in range(3):
                io.foot_sites[f][k] = float(sites[f][k])
        with torch.cuda.device(self.device):
            code = library().duck_servo_substep(self._h, ctypes.byref(params), ctypes.byref(io),
                                                self._stream())
        if code:
            _raise(code, "servo_substep")

    def task_obs_dim(self, task):
        return int(library().duck_task_obs_dim(ctypes.byref(task), self.num_joints))

    def task_targets(self, task, actions, reference, clamped, target, episode=None,
                     commands=None):
        """clamped <- clamp(actions, -1, 1); target <- clamp(ref + scale a, lower, upper)
        with ref = `reference`, else (task.gait) the gait reference of `episode`
        [E] int64 and `commands` [E,2], else HOME."""
        E, J = self.num_envs, self.num_joints
        args = [self._check(actions, [E, J]), self._ptr(reference, [E, J]),
                self._ptr(episode, [E], torch.int64), self._ptr(commands, [E, 2]),
                self._check(clamped, [E, J]), self._check(target, [E, J])]
        with torch.cuda.device(self.device):
            code = library().duck_task_targets(self._h, ctypes.byref(task), *args, self._stream())
        if code:
            _raise(code, "task_targets")

    def task_step(self, task, action, last_action, commands, episode, filtered, returns, obs,
                  reward, failed, timeout, done, diag):
        """Failure, reward, counters and the observation after a physics step."""
        E, J = self.num_envs, self.num_joints
        f32, i64, u8 = torch.float32, torch.int64, torch.bool
        args = [self._check(action, [E, J]), self._check(last_action, [E, J]),
                self._ptr(commands, [E, 2]), self._check(episode, [E], i64),
                self._ptr(filtered, [E, 2]), self._check(returns, [E], f32),
                self._check(obs, [E, self.task_obs_dim(task)], f32),
                self._check(reward, [E], f32), self._check(failed, [E], u8),
                self._check(timeout, [E], u8), self._check(done, [E], u8),
                self._ptr(diag, [E, 6])]
        with torch.cuda.device(self.device):
            code = library().duck_task_step(self._h, ctypes.byref(task), *args, self._stream())
        if code:
            _raise(code, "task_step")

    def task_observe(self, task, reset_mask, actions, commands, episode, filtered, returns,
                     forces, obs):
        """Restart the bookkeeping of `reset_mask` envs, then observe every env."""
        E, J = self.num_envs, self.num_joints
        args = [self._ptr(reset_mask, [E], torch.bool), self._check(actions, [E, J]),
                self._ptr(commands, [E, 2]), self._check(episode, [E], torch.int64),
                self._ptr(filtered, [E, 2]), self._check(returns, [E], torch.float32),
                self._ptr(forces, [E, 3]),
                self._check(obs, [E, self.task_obs_dim(task)], torch.float32)]
        with torch.cuda.device(self.device):
            code = library().duck_task_observe(self._h, ctypes.byref(task), *args, self._stream())
        if code:
            _raise(code, "task_observe")

    def task_reset_inputs(self, task, reset_mask, joint_draws, root_draws, selected, direction,
                          command_speed, commands, q, roots, commands_out):
        """TensorEnv.reset's q [E,J], root offsets [E,6] and, with a command draw
        (`selected` [E] int64 or one `direction` >= 0), commands_out [E,2] from
        the caller's draws, in one launch (duck_task_reset_inputs)."""
        E, J = self.num_envs, self.num_joints
        args = [self._ptr(reset_mask, [E], torch.bool), self._ptr(joint_draws, [E, J]),
                self._ptr(root_draws, [E, 2]), self._ptr(selected, [E], torch.int64),
                int(direction), float(command_speed), self._ptr(commands, [E, 2]),
                self._check(q, [E, J]), self._check(roots, [E, 6]),
                self._ptr(commands_out, [E, 2])]
        with torch.cuda.device(self.device):
            code = library().duck_task_reset_inputs(self._h, ctypes.byref(task), *args,
                                                    self._stream())
        if code:
            _raise(code, "task_reset_inputs")

    # ------------------------------------------------ state introspection
    def state_layout(self):
        out = (ctypes.c_longlong * 51)()
        code = library().duck_state_layout(self._h, out)
        if code:
            _raise(code, "state_layout")
        return list(out)

    def codec(self):
        from .state import StateCodec

        return StateCodec(self.state_layout(), self.num_bodies, self.num_joints)

    def export_state(self):
        """uint8 tensor [E, state_bytes] copy of every environment's HBM state."""
        out = torch.empty(self.num_envs, self.state_bytes, device=self.device, dtype=torch.uint8)
        with torch.cuda.device(self.device):
            code = library().duck_export_state(self._h, ctypes.c_void_p(out.data_ptr()),
                                               self._stream())
        if code:
            _raise(code, "export_state")
        return out

    def import_state(self, raw):
        raw = self._check(raw, [self.num_envs, self.state_bytes], torch.uint8)
        with torch.cuda.device(self.device):
            code = library().duck_import_state(self._h, raw, self._stream())
        if code:
            _raise(code, "import_state")
