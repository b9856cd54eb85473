// CPU oracle for the batched AVBD environment step: TEST INFRASTRUCTURE.
//
// A clean-room restatement of the reference's two solver semantics, used only
// for the expected values in tests/, the bench's cpu_baseline leg and smoke():
//   mode 0  implicit-coloured  = src/cuda/kernel.cuh + convex.cuh + model.hpp
//                                 (what the reference's CudaBatch computes)
//   mode 1  explicit-sequential = src/solver.cpp (explicit PD predictor,
//                                 Gauss-Seidel in body order, ground only)
// in float32 or float64, compiled with -ffp-contract=off.  Every function cites
// the reference lines it restates.  The product never links this library.
//
// All array arguments are float64, whatever the handle's precision.
#pragma once
#ifdef __cplusplus
extern "C" {
#endif
const char *oracle_last_error(void);
void *oracle_create(const char *path, double dt, int iterations, int fp64, int mode);
void oracle_destroy(void *h);
int oracle_dims(void *h, int *bodies, int *joints);
int oracle_reset(void *h, const double *q, const double *root);
int oracle_set_controls(void *h, const double *target, const double *force, double kp,
                        double limit);
int oracle_set_motor(void *h, const double *motor, const double *force);
int oracle_set_friction(void *h, double friction);
int oracle_set_mass_scale(void *h, double scale);
int oracle_set_root_velocity(void *h, const double *v, const double *w);
int oracle_advance(void *h, int substeps);
int oracle_detect(void *h);
int oracle_failed(void *h);
int oracle_snapshot(void *h, double *bodies, double *joints, double *diag);
int oracle_set_body(void *h, int i, const double *x, const double *q, const double *v,
                    const double *w);
int oracle_contacts(void *h, int capacity, int *count, int *ints, double *reals);
int oracle_colors(void *h, int *colors, int *count);
int oracle_joint_state(void *h, double *out);
int oracle_contact_forces(void *h, int ground_only, double *out);
int oracle_self_contact_stats(void *h, double *out);
int oracle_contact_counts(void *h, double *out);
int oracle_generalized_loads(void *h, const double *offset, double *out);
int oracle_convex_query(const double *va, int na, const double *vb, int nb,
                        const double *poses, double inflation, double tolerance, int fp64,
                        double *out);
long long oracle_flops(void);
// The reference's CPU batch (src/cuda/cpu_bindings.cpp:20-168) over mode 0:
// n environments on `threads` env-striped std::thread workers.
void *oracle_batch_create(const char *path, int n, double dt, int iterations, int fp64, int threads);
void oracle_batch_destroy(void *h);
int oracle_batch_dims(void *h, int *n, int *bodies, int *joints);
int oracle_batch_reset(void *h, const unsigned char *mask, const double *q, const double *root);
int oracle_batch_step(void *h, const double *target, const double *forces, int substeps, double kp,
                      double limit);
int oracle_batch_step_motor(void *h, const double *motor, const double *forces);
int oracle_batch_state(void *h, double *bodies, double *joints, double *diag);
int oracle_batch_contact_counts(void *h, double *out);
#ifdef __cplusplus
}
#endif
