/*
 * CPU FP64 oracle of the per-world control step -- TEST INFRASTRUCTURE ONLY.
 *
 * This is the parity oracle and the CPU timing baseline of the MI355X backend.  It restates, in
 * plain serial C++ on doubles, the algorithms of the reference's FP32 control step (each function
 * in oracle.cpp cites the reference file:line it follows).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product path (gpu-libero_amd/) never does.
 *
 * The structs mirror MxModel / MxData of include/mx_physics.h field for field, with double in
 * place of float, so the Python side fills both from the same packed model.
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include "../include/mx_physics.h"

#ifdef __cplusplus
extern "C" {
#endif

#define OR_DECL_DOUBLE(name) double name;
#define OR_DECL_CDOUBLE_PTR(name) const double* name;
#define OR_DECL_DOUBLE_PTR(name) double* name;

typedef struct OrModel {
  MX_MODEL_INT_SCALARS(MX_DECL_INT)
  MX_MODEL_REAL_SCALARS(OR_DECL_DOUBLE)
  MX_MODEL_REAL_ARRAYS(OR_DECL_CDOUBLE_PTR)
  MX_MODEL_INT_ARRAYS(MX_DECL_CINT_PTR)
} OrModel;

typedef struct OrData {
  int32_t nworld;
  int32_t workspace_doubles;   /* unused by the oracle */
  int64_t workspace_total;
  MX_DATA_REAL_ARRAYS(OR_DECL_DOUBLE_PTR)
  MX_DATA_F64_ARRAYS(MX_DECL_F64_PTR)
  MX_DATA_INT_ARRAYS(MX_DECL_INT_PTR)
} OrData;

size_t or_model_bytes(void);
size_t or_data_bytes(void);
int or_field_count(int which);
const char* or_field_name(int which, int index);

/* Same semantics as mx_control_step / mx_forward, on host double arrays; `threads` worker
 * threads (one world at a time per thread), pinned to distinct cores when pin != 0. */
int or_control_step(const OrModel* m, const OrData* d, int substeps, int flags, int threads, int pin);
int or_forward(const OrModel* m, const OrData* d, const int32_t* mask, int flags, int threads);

/* The FP64 operational-space controller alone, on given inputs (for the 1e-9 parity check).
 * n = ndof arm joints (1..8).
 * in: mass[n*n] jac[6*n] q[n] qvel[n] bias[n] ee_pos[3] ee_rot[9] ee_vel[6]  (row-major),
 *     action[7], action_scale[24] (null: OSC_POSE's default ranges), gains[12], q0[n], ctrlrange[2*(n+2)]
 * state (in/out): goal_pos[3] goal_rot[9] gripper[2]
 * out: tau[n] (before clipping), ctrl[n+2], rank[3]; returns the controller error code. */
int or_osc(int ndof, const double* mass, const double* jac, const double* q, const double* qvel,
           const double* bias, const double* ee_pos, const double* ee_rot, const double* ee_vel,
           const double* action, const double* action_scale, const double* gains, const double* q0,
           const double* ctrlrange,
           int uncouple, double gripper_speed, int policy,
           double* goal_pos, double* goal_rot, double* gripper,
           double* tau, double* ctrl, int32_t* rank);

/* One narrowphase call on two geoms given in world frame (geom type, position, row-major
 * rotation, size, mesh vertices in the geom frame and, for meshes, the hull-polygon pack described
 * at unpack_polys in oracle_collision.cpp, or null), with the pair's summed margin and gap, the
 * box-box route (primitive SAT or GJK/EPA) and the CCD options; returns the number of contacts
 * written (pos[3], normal[3] from geom 1 to geom 2, dist), at most maxout, or -1 for an
 * unsupported type pair. */
/* The contact frame of a contact normal (rows: normal, tangent, normal x tangent), as the step
 * builds it for every contact except plane-capsule's. */
void or_contact_frame(const double* normal, double* frame);

int or_collide(int type1, const double* pos1, const double* mat1, const double* size1, const double* vert1,
               int nvert1, const int* poly1, const double* pnorm1, int type2, const double* pos2,
               const double* mat2, const double* size2, const double* vert2, int nvert2, const int* poly2,
               const double* pnorm2, double margin, double gap, int boxbox_primitive,
               double ccd_tolerance, int ccd_iterations, int epa_iterations, double* out_pos,
               double* out_normal, double* out_dist, int maxout);

/* Matrix helpers exposed for golden tests: symmetric Gauss-Jordan inverse and Jacobi pinv. */
int or_spd_inverse(const double* a, int n, double* out);
int or_pinv(const double* a, int n, double* out, int32_t* rank);

#ifdef __cplusplus
}
#endif
#endif
