/* C ABI of the MI355X (gfx950) batched AVBD environment step.
 *
 * Drop-in replacement for the CUDA launch path of the reference batch
 * (src/cuda/extension.cu:160-173 `Interface`, bound to Python as `CudaBatch`
 * at extension.cu:436-452).  The library owns the model and the per-env
 * state in HBM; callers own every input and output buffer.  Device buffers
 * are plain device pointers in the batch dtype (float32, or float64 with
 * fp_bits = 64), C-contiguous with the shapes given below; every call is
 * asynchronous on `hip_stream` (a hipStream_t, NULL = the null stream) and
 * is ordered after the batch's previous call on any stream by a private
 * event, as extension.cu:204-205 orders them.
 *
 * Every function returns 0 on success or a nonzero code; duck_last_error()
 * then describes the failure (thread-local).  Numerical faults of one
 * environment are not errors: they set that environment's diag[5] (failed)
 * until a reset clears it (kernel.cuh:382, 395).
 */
#ifndef DUCK_HIP_H
#define DUCK_HIP_H
#ifdef __cplusplus
extern "C" {
#endif

enum {
  DUCK_OK = 0,
  DUCK_ERR_ARGUMENT = 1, /* invalid argument (TORCH_CHECK in extension.cu) */
  DUCK_ERR_MODEL = 2,    /* model rejected by the flattening checks (model.hpp:5-8) */
  DUCK_ERR_DEVICE = 3,   /* HIP runtime failure */
  DUCK_ERR_RUNTIME = 4   /* unreadable or malformed model file (solver.cpp:67-174) */
};

/* Flags of duck_create. */
#define DUCK_FLAG_SPECIALIZED 1u /* require the MicroDuck 16-body/14-hinge layout */
#define DUCK_FLAG_SPLIT 2u       /* float64: use the float layout (two lanes per body
                                    block solve) instead of one lane per solve */
#define DUCK_FLAG_SHARED_MEMORY 4u /* CudaBatch(shared_memory=True): accepted with
                                      DUCK_FLAG_SPECIALIZED only (extension.cu:424); the
                                      state is always staged in LDS */

/* CudaBatch(model, num_envs, dt, iterations, device, fp64, specialized)
 * (extension.cu:216-265, 423-441).  num_envs in [1, 65536]. */
int duck_create(const char *model_path, int num_envs, double dt, int iterations, int device,
                int fp_bits, unsigned flags, void **out_handle);
/* duck_create on the text of a `.duck` file held in memory (the same checks,
 * messages and error codes; an unparsable text is DUCK_ERR_RUNTIME).  No
 * counterpart in the reference, whose CudaBatch and Solver::load read files:
 * for callers that hold the model in memory, such as duck::Solver, which
 * builds its device batch from its own members without a temporary file. */
int duck_create_text(const char *model_text, int num_envs, double dt, int iterations, int device,
                     int fp_bits, unsigned flags, void **out_handle);
void duck_destroy(void *handle);

/* Parse and validate a `.duck` model file without a device: the checks of
 * duck_create (Solver::load, solver.cpp:67-174; the flattening checks of
 * convert, model.hpp:20-91; the backend checks of makeBatch and the Batch
 * constructor, extension.cu:216-236, 423-435, for `flags`).  out[6] = bodies,
 * joints, shapes, body-contact pairs, ground-contact capacity, body-contact
 * capacity.  Errors as duck_create: DUCK_ERR_RUNTIME for an unreadable or
 * malformed file, DUCK_ERR_MODEL for a flattening or capacity violation,
 * DUCK_ERR_ARGUMENT for the backend's layout checks. */
int duck_model_info(const char *model_path, unsigned flags, int *out);

/* Bodies (including the static world body 0), hinges and contact capacity. */
int duck_dims(void *handle, int *bodies, int *joints, int *contact_capacity);
int duck_num_envs(void *handle);
int duck_fp_bits(void *handle);
/* CudaBatch.joint_names (extension.cu:416-421); valid until duck_destroy. */
const char *duck_joint_name(void *handle, int index);

/* CudaBatch.reset(mask[E] bool, q[E,J], root[E,6]) (extension.cu:273-284):
 * masked re-initialisation and forward kinematics from joint angles and a
 * root (xyz offset, rotation vector).  `ext` (may be NULL) is an [E,5] batch
 * extension with no reference counterpart: ground friction (< 0 keeps the
 * shape friction), mass/inertia scale, initial linear velocity xyz. */
int duck_reset(void *handle, const unsigned char *mask, const void *q, const void *root,
               const void *ext, void *hip_stream);

/* CudaBatch.step(target[E,J], forces[E,3], substeps, kp, limit)
 * (extension.cu:285-306): substeps > 0, kp >= 0, limit >= 0 (0 = uncapped). */
int duck_step(void *handle, const void *target, const void *force, int substeps, double kp,
              double limit, void *hip_stream);

/* CudaBatch.step_motor(motor[E,J,3], forces[E,3]) (extension.cu:307-320):
 * one step with explicit (torque, dry-friction budget, damping) per hinge. */
int duck_step_motor(void *handle, const void *motor, const void *force, void *hip_stream);

/* `substeps` physics steps with the controls each environment's state holds
 * (per-hinge target, kp, torque limit, torque, friction budget, damping, and
 * the root force), as the reference's State::advance (kernel.cuh:421-443)
 * runs them after its callers have set the controls.  No input is read or
 * validated; set the controls through duck_import_state (the C++ duck::Solver
 * does).  substeps > 0. */
int duck_advance(void *handle, int substeps, void *hip_stream);

/* CudaBatch.state() (extension.cu:321-335): bodies[E,B,13] (COM xyz, wxyz,
 * v, w), joints[E,J,2] (angle, rate), diag[E,6] (joint error, penetration,
 * contacts, converged, axis error, failed). */
int duck_state(void *handle, void *bodies, void *joints, void *diag, void *hip_stream);

/* CudaBatch.contact_forces(ground_only) -> [E,B,3] (extension.cu:336-347). */
int duck_contact_forces(void *handle, int ground_only, void *out, void *hip_stream);
/* CudaBatch.self_contact_stats() -> [E,2] (extension.cu:348-359). */
int duck_self_contact_stats(void *handle, void *out, void *hip_stream);
/* CudaBatch.contact_counts() -> [E,2] (extension.cu:360-370). */
int duck_contact_counts(void *handle, void *out, void *hip_stream);
/* CudaBatch.generalized_loads(offset[E,3]) -> [E,J,3] (extension.cu:371-384). */
int duck_generalized_loads(void *handle, const void *offset, void *out, void *hip_stream);

/* CudaBatch.reference(target[J], forces[3], substeps, kp, limit)
 * (extension.cu:385-415): one environment advanced from the model file's
 * initial state; host pointers in the batch dtype.  Synchronous.  Computed on
 * the batch's device with the same kernels (this library carries no CPU
 * solver). */
int duck_reference(void *handle, const void *target, const void *force, int substeps, double kp,
                   double limit, void *bodies, void *joints, void *diag);

/* duck_reference without any allocation.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  The state blob
 * and the device copies of the inputs and outputs live in the library's
 * static device scratch, 64 KiB per device (held until the process ends);
 * a model whose blob plus 6 + 3 J + 13 B reals exceeds it is rejected with
 * DUCK_ERR_ARGUMENT.  Results are those of duck_reference.  The scratch is
 * shared by every call on a device and keeps the last call's contents;
 * calls on one device are serialised by a host lock held for the whole call
 * (calls from several host threads take turns). */
int duck_reference_noalloc(void *handle, const void *target, const void *force, int substeps,
                           double kp, double limit, void *bodies, void *joints, void *diag);

/* Resources of the kernel that duck_step (which = DUCK_KERNEL_STEP) or
 * duck_servo_substep (DUCK_KERNEL_SERVO_SUBSTEP) launches for this batch (no
 * reference counterpart: for measurement).  out[7] = VGPRs per lane, static
 * LDS bytes per workgroup, scratch bytes per lane, resident workgroups per CU
 * (the runtime's occupancy calculator), lanes per workgroup, environments per
 * workgroup, workgroups per launch.  Waves per SIMD = workgroups per CU x
 * lanes per workgroup / 64 / 4. */
enum { DUCK_KERNEL_STEP = 0, DUCK_KERNEL_SERVO_SUBSTEP = 1 };
int duck_kernel_info(void *handle, int which, long long *out);

/* Size in bytes of one environment's HBM state blob. */
long long duck_state_bytes(void *handle);

/* State introspection (no reference counterpart: the reference keeps its
 * state opaque).  For tests that compare the full per-env state with the CPU
 * oracle and that seed identical states.  duck_state_layout writes 51
 * int64 values: capacities B J CG CS, scalar bytes, blob bytes, header bytes,
 * the byte offsets of the EnvState fields x q v w mass inertia force lambda
 * penalty lambdaF penaltyF target kp maxTorque torque frictionloss damping
 * diag friction failed ngc nsc colors colorCount gc, ground-contact bytes, the
 * offset of sc, self-contact bytes, then the field offsets of a ground contact
 * (id local anchor c0 lambda penalty) and of a self contact (id local localB
 * t1 t2 n c0 friction lambda penalty).  Export/import copy all E blobs
 * (E * duck_state_bytes bytes) to/from a device buffer. */
int duck_state_layout(void *handle, long long *out);
int duck_export_state(void *handle, void *dst, void *hip_stream);
int duck_import_state(void *handle, const void *src, void *hip_stream);

/* ---- Control step of the tensor VecEnv (python/duck_gym/tensor_env.py) ----
 * The reference assembles targets, observations, rewards and terminations
 * from ~40 torch ops per control step (tensor_env.py:178-219, 221-391); here
 * they are three kernels that read the HBM state directly. */
#define DUCK_MAX_JOINTS 32
enum {
  DUCK_TASK_STANDING = 0,   /* tensor_env.py task="standing": 52-wide observation */
  DUCK_TASK_LOCOMOTION = 1, /* task="locomotion": 58 (+2 with the velocity filter) */
  DUCK_TASK_ROLLOUT = 2     /* 48-wide observation (gravity, w, q-HOME, 0.1 qdot, action),
                               locomotion reward, failure = base height below fall_height */
};
typedef struct DuckTask {
  int kind;            /* DUCK_TASK_* */
  int velocity_filter; /* locomotion: velocity_filter_seconds > 0 */
  double home[DUCK_MAX_JOINTS], lower[DUCK_MAX_JOINTS], upper[DUCK_MAX_JOINTS];
  double iquat[4];     /* metadata root_iquat (w x y z); the root frame is q_body1 * conj(iquat) */
  double root_height, action_scale, control_dt, gait_period;
  double tracking_weight, heading_weight, tracking_sigma, velocity_alpha;
  double fall_height;
  long long max_episode_length;
  /* Gait-table options (tensor_env.py:151-170, 263-277, 328-354), all zero when off.
   * gait: the servo reference blends HOME into the table row of the command's
   * direction (duck_task_targets); foot_clearance / load_transfer: the two
   * shaping terms of the reward (duck_task_step). */
  int gait, foot_clearance, load_transfer;
  int gait_phases;         /* phases per direction in gait_table */
  const void *gait_table;  /* [4, gait_phases, J] batch dtype, device (gait) */
  double gait_lift;        /* foot_clearance: the swing foot's lift */
  int feet[2];             /* the two foot bodies (foot_clearance, load_transfer) */
  int foot_points;         /* body-frame collision points per foot */
  const void *foot_point;  /* [2, foot_points, 3] batch dtype, device (foot_clearance) */
  double weight;           /* load_transfer: metadata mass x 9.81 */
} DuckTask;

/* Observation width of `task` for a batch with `joints` hinges. */
int duck_task_obs_dim(const DuckTask *task, int joints);

/* TensorEnv.step head (tensor_env.py:279-283, 263-277): a = clamp(actions,-1,1),
 * target = clamp(ref + action_scale a, lower, upper).  ref: `reference` [E,J]
 * when not NULL; else, with task->gait, the gait reference of the episode
 * counters `episode` [E] int64 and `commands` [E,2]; else HOME.  [E,J] batch
 * dtype. */
int duck_task_targets(void *handle, const DuckTask *task, const void *actions,
                      const void *reference, const long long *episode, const void *commands,
                      void *clamped, void *target, void *hip_stream);

/* TensorEnv.step tail after the physics (tensor_env.py:345-391): failure,
 * reward, returns, episode counters, timeouts, done, the observation of the
 * new state and diag[E,6].  `action` [E,J] is this step's clamped action;
 * `last_action` [E,J] holds the previous one and is overwritten with `action`.
 * commands [E,2] (locomotion/rollout, else NULL), episode [E] int64, filtered
 * [E,2] (velocity filter, else NULL), returns/obs/reward float32, failed /
 * timeout / done [E] bytes.  With task->foot_clearance / load_transfer the
 * shaping terms join the reward before the failure and the control period
 * apply (tensor_env.py:328-355). */
int duck_task_step(void *handle, const DuckTask *task, const void *action, void *last_action,
                   const void *commands, long long *episode, void *filtered, float *returns,
                   float *obs, float *reward, unsigned char *failed, unsigned char *timeout,
                   unsigned char *done, void *diag, void *hip_stream);

/* TensorEnv.reset's inputs (tensor_env.py:196-217) in one launch, from the
 * random draws the caller made on its generator in the reference's order:
 * q [E,J] = HOME + (u - 0.5) * 0.02 with u = joint_draws [E,J] (HOME when
 * NULL); roots [E,6] = (0, 0, 0.001, (v - 0.5) * 0.02, 0) with v = root_draws
 * [E,2] (zeros when NULL); with a command draw, `selected` [E] int64 or one
 * `direction` (0-3) for every env (-1 and NULL: none), commands_out [E,2] =
 * reset_mask ? table[direction] * command_speed : commands, the table
 * [[1, 0], [-1, 0], [0, 1], [0, -1]].  Each value is rounded per operation, as
 * the reference's torch expressions are.  Batch dtype.  No counterpart in the
 * reference, which spends about a dozen torch launches on these. */
int duck_task_reset_inputs(void *handle, const DuckTask *task, const unsigned char *reset_mask,
                           const void *joint_draws, const void *root_draws,
                           const long long *selected, int direction, double command_speed,
                           const void *commands, void *q, void *roots, void *commands_out,
                           void *hip_stream);

/* TensorEnv.reset bookkeeping + get_observations (tensor_env.py:199-219, 259):
 * for envs in `reset_mask` (may be NULL) zero the actions, filtered velocity,
 * forces [E,3] (may be NULL), episode counter and return; then write the
 * observation of every env. */
int duck_task_observe(void *handle, const DuckTask *task, const unsigned char *reset_mask,
                      void *actions, const void *commands, long long *episode, void *filtered,
                      float *returns, void *forces, float *obs, void *hip_stream);

/* ---- BAM servo substep (python/duck_gym/bam_env.py:307-326) ----
 * Parameters of the XL330/m6 actuator equations (python/duck_gym/actuator.py:
 * 16-77; names as in the BAM parameter dictionary and the official config). */
typedef struct DuckServo {
  double kt, resistance, dtheta_stribeck, alpha, friction_base, friction_stribeck;
  double load_friction_external, load_friction_motor, load_friction_external_stribeck;
  double load_friction_motor_stribeck, load_friction_external_quad, load_friction_motor_quad;
  double friction_viscous;
  double vin, vin_drop_gain, vin_min, kp_fw, kp_scale, kd_scale, friction_scale, force_limit;
  int lag; /* actuator delay in physics steps; the ring holds lag + 1 targets */
} DuckServo;

/* One servo substep before duck_step_motor: history[cursor] = target (every
 * slot for envs whose `initialized` flag is 0, which is then set), delayed =
 * history[(cursor - lag) mod (lag + 1)]; external hinge load = -bias +
 * constraint of the Newton-Euler pass with root COM offset `root_offset`
 * [E,3] (duck_generalized_loads columns 0 and 1); the XL330 model gives
 * motor [E,J,3] = (clamped torque, friction budget, damping), and
 * previous_motor / previous_applied [E,J] are replaced by this substep's raw /
 * clamped torque.  history [lag+1,E,J]; supply [E] may be NULL.  The caller
 * advances `cursor` = (cursor + 1) mod (lag + 1) per substep. */
int duck_servo(void *handle, const DuckServo *servo, const void *target, void *history,
               int cursor, unsigned char *initialized, const void *root_offset,
               void *previous_motor, void *previous_applied, void *motor, void *supply,
               void *hip_stream);

#define DUCK_MAX_FEET 4

/* Buffers and frame data of one fused servo substep (duck_servo_substep).
 * All real buffers are in the batch dtype; the optional ones may be NULL. */
typedef struct DuckServoSubstep {
  const void *target;           /* [E,J] targets of this control step */
  void *history;                /* [lag+1,E,J] ring of targets */
  int cursor;                   /* slot this substep writes */
  unsigned char *initialized;   /* [E] ring filled since the last reset */
  const void *root_offset;      /* [E,3] root COM offset (load pass, origin velocity) */
  void *previous_motor;         /* [E,J] raw motor torque of the last substep, in/out */
  void *previous_applied;       /* [E,J] clamped torque of the last substep, in/out */
  void *motor;                  /* [E,J,3] motor channels of this substep, out */
  void *supply;                 /* [E] supply voltage, out */
  void *self_contacts;          /* [E] running maximum of active body contacts, in/out */
  void *self_penetration;       /* [E] running maximum of body-contact depth, in/out */
  double root_principal_quat[4]; /* (w, x, y, z): root frame = body 1 frame * its conjugate */
  int num_feet;                 /* 0 .. DUCK_MAX_FEET */
  int foot_bodies[DUCK_MAX_FEET];
  double foot_sites[DUCK_MAX_FEET][3]; /* foot site in its body's frame */
  void *gravity;                /* [E,3] gravity direction in the root frame, out */
  void *angular_velocity;       /* [E,3] root angular velocity in the root frame, out */
  void *linear_velocity;        /* [E,3] root-origin velocity in the root frame, out */
  void *origin_velocity;        /* [E,3] root-origin velocity in the world, out */
  void *foot_forces;            /* [E,F,3] ground contact force on each foot body, out */
  void *site_positions;         /* [E,F,3] foot sites in the world, out */
  void *site_velocities;        /* [E,F,3] foot site velocities, out */
  void *air_time;               /* [E,F] seconds since the foot last touched, in/out */
  void *contact_time;           /* [E,F] seconds the foot has touched, in/out */
  void *mean_velocity;          /* [E,3] low-passed root-origin world velocity, in/out
                                   (NULL = no filter; bam_env.py:343-345) */
  double mean_velocity_alpha;   /* filter weight per substep, -expm1(-dt / tau) */
} DuckServoSubstep;

/* One substep of the BAM-actuated environment in one launch
 * (python/duck_gym/bam_env.py:307-337 with refresh(), bam_env.py:128-155):
 * the servo substep of duck_servo, the motor step of duck_step_motor with a
 * zero root force, then the self-contact statistics folded into their
 * running maxima (bam_env.py:333-335) and the quantities refresh() derives
 * from the new state: gravity and velocities in the root frame, the ground
 * contact force on each foot (duck_contact_forces with ground_only), foot
 * site positions and velocities, and the air/contact timers (a foot touches
 * when its force exceeds 1e-5 N).  With `mean_velocity`, the filter of
 * bam_env.py:343-345 follows: mean += alpha (origin_velocity - mean), in
 * that operation order.  The caller advances `cursor` per
 * substep as for duck_servo.  No reference counterpart as one call: it
 * replaces the reference loop's five calls and torch arithmetic. */
int duck_servo_substep(void *handle, const DuckServo *servo, const DuckServoSubstep *io,
                       void *hip_stream);

/* ---- Explicit-sequential step (src/solver.cpp:315-537) ----
 * The step of the reference's independent float64 solver, duck::Solver::step
 * (include/duck/solver.hpp:56-80): the PD drive as an explicit torque in the
 * predictor (solver.cpp:339-347), block Gauss-Seidel over the bodies in index
 * order (solver.cpp:363), ground contacts only (solver.cpp:216-302), the
 * hinges' angle0 / velocity0 / c0 kept, and the diagnostics including the
 * largest block update.  The structs mirror duck::Options, Body, Joint,
 * Shape, Contact and Diagnostics field for field (vectors as [3], quaternions
 * as w x y z); duck::Solver::step and duck::Batch::step fill them. */
typedef struct DuckSeqOptions {
  double dt, alpha, gamma, beta_linear, beta_angular, tolerance, gravity[3];
  int iterations, ground;
} DuckSeqOptions;
typedef struct DuckSeqBody {
  double mass, inertia[3], x[3], v[3], w[3], x0[3], xp[3], force[3], q[4], q0[4], qp[4];
} DuckSeqBody;
typedef struct DuckSeqJoint {
  int a, b, limited, reserved;
  double ra[3], rb[3], axis_a[3], axis_b[3], tangent_a[3], tangent_b[3];
  double lo, hi, damping, armature, frictionloss, lambda_f, penalty_f, torque, kp, target,
      max_torque, angle0, velocity0, lambda[7], penalty[7], c0[7];
} DuckSeqJoint;
typedef struct DuckSeqShape {
  int body, type, ground;
  int first_point, num_points; /* its body-frame candidate points (Shape::localPoints) in
                                  DuckSeqEnv.points */
  double center[3], size[3], q[4], friction, bounding_radius;
} DuckSeqShape;
typedef struct DuckSeqContact {
  int body, shape, feature, stick;
  double local[3], anchor[3], radius, friction, c0, lambda[3], penalty[3];
} DuckSeqContact;
typedef struct DuckSeqDiagnostics {
  double joint_error, axis_error, penetration, update;
  int contacts, iterations, converged, reserved;
} DuckSeqDiagnostics;
enum {
  DUCK_SEQ_OK = 0,
  DUCK_SEQ_HESSIAN = 1,    /* "Non-positive local Hessian" (math.hpp:91) */
  DUCK_SEQ_NONFINITE = 2,  /* "Non-finite state" (solver.cpp:521) */
  DUCK_SEQ_QUATERNION = 3  /* "Zero quaternion" (math.hpp:53) */
};
typedef struct DuckSeqEnv {
  DuckSeqOptions options;
  int num_bodies, num_joints, num_shapes, num_points;
  int num_contacts;     /* in: the contacts of the last step; out: this step's */
  int contact_capacity; /* entries of `contacts`: at least num_contacts and 4 per shape */
  DuckSeqBody *bodies;
  DuckSeqJoint *joints;
  const DuckSeqShape *shapes;
  const double *points; /* [num_points][3] */
  DuckSeqContact *contacts;
  DuckSeqDiagnostics diagnostics; /* out */
  int status;                     /* out: DUCK_SEQ_*; the environment stops at a fault */
} DuckSeqEnv;

/* `steps` steps of each of `num_envs` independent environments (host
 * structs, updated in place), one GPU thread per environment on `device`;
 * synchronous.  Argument errors return DUCK_ERR_ARGUMENT and change nothing:
 * the reference's "Invalid solver options" (solver.cpp:318-320), an index out
 * of range, a capacity below the step's needs, or more than 2e5 iterations x
 * steps in one call (a bound on the kernel's running time: one thread runs an
 * environment's iterations serially).
 * A numerical fault of one environment is its `status`, where the reference
 * throws, and leaves that environment as the reference's step leaves it when
 * it throws. */
int duck_sequential_step(DuckSeqEnv *envs, int num_envs, int steps, int device);

const char *duck_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
