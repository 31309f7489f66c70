/*
 * mx_physics.h -- C ABI of the MI355X-native batched physics backend (libmx_physics.so).
 *
 * The library replaces the reference's per-world control step, which the reference exposes as
 * ~30 leaf libraries with the convention
 *     extern "C" int flash_<leaf>_launch(const <Leaf>Inputs*, [int stage,] cudaStream_t)
 *     size_t flash_<leaf>_arguments_bytes(); int flash_<leaf>_arch(); const char* flash_<leaf>_source_id();
 * (e.g. gpu/cuda/newton/mjwarp_solver_state.cu:138-159, gpu/cuda/newton/mjwarp_linesearch.cu:377-407,
 *  bound by ctypes in gpu/host/runtime/dynamics/mjwarp_motion.py:20-37).
 * Here the whole control step is one world-local entry point, and the same ABI-check convention is
 * kept: argument-struct sizes, the target architecture and a source id are exported for the loader.
 *
 * Conventions (as in the reference leaves):
 *   - every pointer is a device pointer owned by the caller; the library never allocates;
 *   - the argument structs are read on the host and copied by value into the kernel launch;
 *   - per-world arrays are world-major: field[w * width + k];
 *   - return value 0 = success, > 0 = HIP error code, < 0 = MX_ERR_* (invalid argument or a model
 *     outside the admitted domain), detected before any launch;
 *   - per-world numerical failures are data (overflow bits, controller error), not return codes.
 * Streams are passed as void* (a hipStream_t); a null stream is the default stream.
 */
#ifndef MX_PHYSICS_H
#define MX_PHYSICS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MX_ABI_VERSION 18

#define MX_ERR_INVALID   (-1)   /* null pointer, bad dimension or struct */
#define MX_ERR_DOMAIN    (-2)   /* model outside the admitted domain (sizes, joint types) */
#define MX_ERR_LDS       (-3)   /* working set exceeds the LDS budget and no workspace is given */
#define MX_ERR_SCRATCH   (-4)   /* mx_control_step_noalloc: the batch needs more than MX_SCRATCH_BYTES */

/* Bytes of the fixed device scratch behind mx_control_step_noalloc (64 MiB, one copy per device). */
#define MX_SCRATCH_BYTES (64u << 20)

/* The operational-space controller drives osc_ndof arm joints (1 <= osc_ndof <= MX_OSC_MAXDOF) and
 * two gripper actuators; its per-world arrays are sized by osc_ndof (osc_mass n*n, osc_jac 6*n,
 * osc_q / osc_qvel / osc_bias / osc_q0 / osc_tau n); the action stays 7 (pose delta, gripper). */
#define MX_OSC_MAXDOF 8

/* Action scaling of the pose delta (robosuite Controller.scale_action; the reference's optional
 * action_config, gpu/cuda/control/osc_solver.cu:38-47, gpu/host/runtime/control/__init__.py:65-74).
 * With the model scalar osc_action_scaled = 0, robosuite OSC_POSE's default ranges apply: action
 * component k in [-1, 1] maps to 0.05 m (k < 3) or 0.5 rad (k = 3..5) per unit.  With 1, each
 * world's 24 doubles of osc_action_scale hold input_min[6], input_max[6], output_min[6], output_max[6]
 * (input_min < input_max), and component k is clip(a, in_min, in_max) - (in_max + in_min) / 2,
 * times |out_max - out_min| / |in_max - in_min|, plus (out_max + out_min) / 2.  At a policy substep
 * the goal position becomes ee_pos + delta[0:3]; the goal orientation becomes R(delta[3:6]) ee_rot
 * when some rotation component is nonzero and is kept otherwise (robosuite's set_goal). */
#define MX_OSC_ACTION_SCALE 24

/* LDS of one workgroup on gfx950.  A model whose per-world working set (mx_lds_bytes) exceeds it
 * runs with that working set in the caller's `workspace` array instead (mx_workspace_bytes). */
#define MX_LDS_BUDGET 163840

/* Overflow bits per world (reference gpu/host/backends/cuda_fp32/constants.py:70-102). */
#define MX_OVERFLOW_NEFC          (1 << 0)
#define MX_OVERFLOW_BROADPHASE    (1 << 2)
#define MX_OVERFLOW_NARROWPHASE   (1 << 3)
#define MX_OVERFLOW_CCD           (1 << 4)
#define MX_OVERFLOW_EPA_HORIZON   (1 << 8)
#define MX_OVERFLOW_ITERATIONS    (1 << 9)
#define MX_OVERFLOW_LS_ITERATIONS (1 << 10)
/* No counterpart in the reference (bits 0-11 are its own): the kernel could not locate its launch
   parameters (a compiler placing the hidden kernel arguments elsewhere); nothing was computed. */
#define MX_OVERFLOW_LAUNCH        (1 << 12)

/* Controller error codes (reference gpu/cuda/control/osc_solver.cu:443-446,477-483). */
#define MX_OSC_CACHE_INVALID 1
#define MX_OSC_SINGULAR_MASS 2
#define MX_OSC_PINV_FAILED   4

/* Launch flags for mx_control_step / mx_forward. */
#define MX_FLAG_POLICY_FIRST 1   /* first substep is a policy step (OSC goal update) */
#define MX_FLAG_NO_CONTROL   2   /* skip the OSC (ctrl kept as given)                  */
#define MX_FLAG_NO_INTEGRATE 4   /* forward only: no Euler step                        */
#define MX_FLAG_BOOTSTRAP    8   /* set the OSC goal to the current end-effector pose  */
#define MX_FLAG_WORKSPACE   16   /* working set in `workspace` (the default for models with rows when a workspace is given) */
#define MX_FLAG_LDS         32   /* working set in LDS even when a workspace is given (if it fits) */
/* The FP64 route: the physics computed in double (the reference's FP64 precision route,
 * gpu/host/backends/selection.py:12-16, physics_engine "native" at precision "fp64"), with the
 * working set in LDS; MX_ERR_LDS when mx_lds_bytes_fp64(model) exceeds the workgroup's LDS.  The
 * model arena and the MxData fields stay FP32 (state enters and leaves rounded to float), the
 * controller is the FP64 OSC of every route.  Ignores MX_FLAG_WORKSPACE and MX_FLAG_LDS. */
#define MX_FLAG_FP64        64

/* Sensors: force (MX_SENS_FORCE) and torque (MX_SENS_TORQUE) sensors at a site, three values each
 * at sensordata[sensor_adr], in the site frame (reference gpu/cuda/dynamics/mjwarp_queries.cu:31;
 * the reference admits exactly these two types, gpu/host/backends/cuda_fp32/model.py:39,143).
 * sensor_datatype 0 clips to [-cutoff, cutoff], 1 to (-inf, cutoff]; cutoff 0 does not clip. */
#define MX_SENS_FORCE  4
#define MX_SENS_TORQUE 5

/* ---------------------------------------------------------------- model arrays (per model) */
/* Real-valued model arrays: float on the device, double in the CPU oracle. */
#define MX_MODEL_REAL_ARRAYS(X) \
  X(body_pos) X(body_quat) X(body_ipos) X(body_iquat) X(body_mass) X(body_subtreemass) \
  X(body_inertia) X(body_invweight0) \
  X(jnt_pos) X(jnt_axis) X(jnt_range) X(jnt_stiffness) X(jnt_margin) X(jnt_solref) X(jnt_solimp) \
  X(qpos0) X(qpos_spring) \
  X(dof_armature) X(dof_damping) X(dof_frictionloss) X(dof_invweight0) X(dof_solref) X(dof_solimp) \
  X(geom_pos) X(geom_quat) X(geom_size) X(geom_rbound) X(geom_aabb) X(geom_friction) \
  X(geom_solref) X(geom_solimp) X(geom_solmix) X(geom_margin) X(geom_gap) \
  X(site_pos) X(site_quat) X(mesh_vert) X(mesh_polynormal) \
  X(actuator_gear) X(actuator_gainprm) X(actuator_biasprm) X(actuator_ctrlrange) X(actuator_forcerange) \
  X(body_gravcomp) X(sensor_cutoff)

#define MX_MODEL_INT_ARRAYS(X) \
  X(body_parent) X(body_rootid) X(body_weldid) X(body_treeid) X(body_jntadr) X(body_jntnum) \
  X(body_dofadr) X(body_dofnum) X(body_subtreesize) X(body_lastdof) X(level_adr) X(level_body) \
  X(jnt_type) X(jnt_body) X(jnt_qposadr) X(jnt_dofadr) X(jnt_limited) \
  X(dof_body) X(dof_jnt) X(dof_parent) X(dof_treeid) \
  X(tree_dofadr) X(tree_dofnum) X(tree_madr) X(tree_dampadr) X(mpair_i) X(mpair_j) \
  X(geom_type) X(geom_body) X(geom_contype) X(geom_conaffinity) X(geom_condim) X(geom_priority) \
  X(geom_dataid) X(site_body) X(mesh_vertadr) X(mesh_vertnum) \
  X(mesh_polynum) X(mesh_polyadr) X(mesh_polyvertadr) X(mesh_polyvertnum) X(mesh_polyvert) \
  X(mesh_polymapadr) X(mesh_polymapnum) X(mesh_polymap) \
  X(actuator_trnid) X(actuator_biastype) X(actuator_ctrllimited) X(actuator_forcelimited) \
  X(pair_geom) X(osc_qposadr) X(osc_dofadr) X(osc_actuator) \
  X(jnt_actgravcomp) X(sensor_type) X(sensor_objid) X(sensor_adr) X(sensor_datatype)

/* Scalars of the model, in one block so that the float and double variants share a layout. */
#define MX_MODEL_INT_SCALARS(X) \
  X(abi_version) X(nq) X(nv) X(nu) X(nbody) X(njnt) X(ngeom) X(nsite) X(nmesh) X(nmeshvert) \
  X(npair) X(ntree) X(nM) X(nMpair) X(nlevel) X(nconmax) X(njmax) \
  X(opt_iterations) X(opt_ls_iterations) X(opt_cone) X(opt_disableflags) \
  X(osc_site) X(osc_uncouple) X(has_body_active) X(maxchain) X(maxtree) X(maxpairdof) \
  X(opt_ccd_iterations) X(epa_iterations) X(boxbox_primitive) \
  X(nsensor) X(nsensordata) X(has_gravcomp) X(has_fluid) X(nMdamp) X(osc_ndof) X(convex_mpr) X(opt_mpr_iterations) \
  X(osc_action_scaled)

#define MX_MODEL_REAL_SCALARS(X) \
  X(opt_timestep) X(opt_tolerance) X(opt_ls_tolerance) X(opt_impratio) \
  X(opt_gravity_x) X(opt_gravity_y) X(opt_gravity_z) X(osc_gripper_speed) X(meaninertia) \
  X(opt_ccd_tolerance) X(opt_density) X(opt_viscosity) X(opt_wind_x) X(opt_wind_y) X(opt_wind_z) X(opt_mpr_tolerance)

/* ---------------------------------------------------------------- data arrays (per world) */
/* Real-valued per-world arrays: float on the device, double in the CPU oracle.              */
#define MX_DATA_REAL_ARRAYS(X) \
  X(time) X(qpos) X(qvel) X(ctrl) X(qacc_warmstart) X(qfrc_applied) \
  X(qacc) X(qacc_smooth) X(qfrc_bias) X(qfrc_passive) X(qfrc_actuator) X(qfrc_smooth) \
  X(qfrc_constraint) X(actuator_force) X(M) \
  X(xpos) X(xquat) X(xmat) X(geom_xpos) X(geom_xmat) X(site_xpos) X(site_xmat) X(subtree_com) \
  X(osc_mass) X(osc_jac) X(osc_q) X(osc_qvel) X(osc_bias) X(osc_ee_pos) X(osc_ee_rot) X(osc_ee_vel) \
  X(contact_pos) X(contact_frame) X(contact_dist) X(contact_friction) X(contact_includemargin) \
  X(efc_force) X(efc_pos) X(efc_D) X(efc_aref) \
  X(xfrc_applied) X(cacc) X(cfrc_int) X(cfrc_ext) X(sensordata)

/* FP64 per-world arrays (the controller's FP64 section), double in both implementations.
 * stat_sums (4 per world): over every substep computed since the caller last cleared it, the
 * sums of the constraint rows, the contacts, the Newton iterations and iterations x rows (models
 * with constraint rows; the counts the algorithmic-bytes figure of a benchmark averages).        */
#define MX_DATA_F64_ARRAYS(X) \
  X(osc_action) X(osc_goal_pos) X(osc_goal_rot) X(osc_gripper) X(osc_gains) X(osc_q0) X(osc_tau) \
  X(osc_action_scale) X(stat_sums) X(workspace)

#define MX_DATA_INT_ARRAYS(X) \
  X(overflow) X(osc_error) X(osc_rank) X(nstep) X(body_active) \
  X(ncon) X(contact_geom) X(contact_dim) X(nefc) X(efc_type) X(efc_state) X(efc_id) X(solver_niter)

/* ---------------------------------------------------------------- structs */
#define MX_DECL_INT(name) int32_t name;
#define MX_DECL_FLOAT(name) float name;
#define MX_DECL_CFLOAT_PTR(name) const float* name;
#define MX_DECL_CINT_PTR(name) const int32_t* name;
#define MX_DECL_FLOAT_PTR(name) float* name;
#define MX_DECL_F64_PTR(name) double* name;
#define MX_DECL_INT_PTR(name) int32_t* name;

/* Model: sizes, options and device pointers to the model arrays (float). */
typedef struct MxModel {
  MX_MODEL_INT_SCALARS(MX_DECL_INT)
  MX_MODEL_REAL_SCALARS(MX_DECL_FLOAT)
  MX_MODEL_REAL_ARRAYS(MX_DECL_CFLOAT_PTR)
  MX_MODEL_INT_ARRAYS(MX_DECL_CINT_PTR)
} MxModel;

/* Data: device pointers to the per-world arrays of nworld worlds. */
typedef struct MxData {
  int32_t nworld;
  int32_t workspace_doubles;   /* per-world width of `workspace` in doubles (0: no workspace) */
  int64_t workspace_total;     /* doubles allocated at `workspace` (>= (nworld + 1) * width) */
  MX_DATA_REAL_ARRAYS(MX_DECL_FLOAT_PTR)
  MX_DATA_F64_ARRAYS(MX_DECL_F64_PTR)
  MX_DATA_INT_ARRAYS(MX_DECL_INT_PTR)
} MxData;

/* ---------------------------------------------------------------- observation plan */
/* An ordered robosuite observable plan sampled on the device (reference
 * gpu/cuda/fp32/fused_observations.cu:39-168 pack_and_sample, gpu/host/backends/cuda_fp32/
 * observations.py:19-110 DeviceObservations, plan schema gpu/host/adapters/observations/schema.py).
 * Spec s writes size[s] floats at offset[s] of each world's `width` floats.  Operations: */
#define MX_OBS_GATHER         0   /* value j = source[indices[index_offset + j]] (MX_OBS_SRC << 24 | element) */
#define MX_OBS_COS            1   /* cos of the dependency's values (dep0: its offset)                        */
#define MX_OBS_SIN            2   /* sin of the dependency's values                                            */
#define MX_OBS_INVERSE_POSE   3   /* 4x4 inverse of the pose (dep0: position, dep1: quaternion x y z w)        */
#define MX_OBS_RELATIVE_POS   4   /* position of a pose (dep0, dep1) in the frame of a 4x4 pose (dep2); its   */
                                  /* quaternion is kept aside for MX_OBS_RELATIVE_QUAT                          */
#define MX_OBS_RELATIVE_QUAT  5   /* the quaternion kept by the MX_OBS_RELATIVE_POS spec at dep0               */
/* Gather sources (bits 24..31 of an index; the element in bits 0..23). */
#define MX_OBS_SRC_QPOS  0
#define MX_OBS_SRC_QVEL  1
#define MX_OBS_SRC_SITE_XPOS 2
#define MX_OBS_SRC_XPOS  3
#define MX_OBS_SRC_XQUAT 4
/* presence[3 s + i]: the spec whose presence the operation's dependency i requires.  Clocks follow
 * the reference: each sampling call adds dt to a spec's elapsed time; a spec samples when not yet
 * sampled in its period and period >= elapsed, when forced, or when its period is due and it has
 * not sampled; a due period wraps elapsed (fmod) and clears `sampled`.  Per-world state arrays are
 * world-major: cache, observed, sidequat (nworld x width), elapsed, sampled, present, events
 * (nworld x nspec).  At most MX_OBS_MAX_SPECS specs. */
#define MX_OBS_MAX_SPECS 128
typedef struct MxObsPlan {
  int32_t nspec, width;
  const int32_t *op, *offset, *size, *index_offset, *indices, *dep0, *dep1, *dep2, *presence, *enabled;
  const float* period;
  float *cache, *observed, *sidequat, *elapsed;
  int32_t *sampled, *present, *events;
} MxObsPlan;

/* ---------------------------------------------------------------- entry points */

/* ABI checks, as flash_<leaf>_arguments_bytes/arch/source_id (gpu/cuda/newton/mjwarp_solver_state.cu:138-141). */
int mx_abi_version(void);
size_t mx_model_bytes(void);                 /* sizeof(MxModel) */
size_t mx_data_bytes(void);                  /* sizeof(MxData)  */
int mx_arch(void);                           /* 950 for gfx950  */
const char* mx_source_id(void);
/* Field tables: which = 0 model real arrays, 1 model int arrays, 2 model int scalars,
 * 3 model real scalars, 4 data real arrays, 5 data f64 arrays, 6 data int arrays. */
int mx_field_count(int which);
const char* mx_field_name(int which, int index);

/* Admission: validates sizes and pointers, returns 0 or MX_ERR_*. Called by every launch entry.
 * Pointers checked: every model array; every per-world state, derived and controller array; when
 * njmax > 0 also the contact, row and count arrays, and body_active when has_body_active.
 * Mirrors the reference admission checks before capture (gpu/host/backends/cuda_fp32/model.py:30-41). */
int mx_check(const MxModel* model, const MxData* data);

/* LDS bytes per world the step kernel uses for this model (for reporting and admission). */
int mx_lds_bytes(const MxModel* model);

/* The same for the FP64 route (MX_FLAG_FP64): the working set with every physics value in double.
 * No counterpart in the reference's FP32 interface; its FP64 route keeps the state in device arrays. */
int mx_lds_bytes_fp64(const MxModel* model);

/* Per-world bytes of the `workspace` array (a multiple of 256) for this model: the working set of
 * one world when it lives in device memory, as the reference keeps its Newton workspace in device
 * arrays (gpu/host/backends/cuda_fp32/data.py:22-70 newton_workspace).  data->workspace then holds
 * (nworld + 1) * data->workspace_doubles doubles with workspace_doubles * 8 >= this value: one slab
 * per world plus slab 0, where each launch writes the model image that all its worlds read.
 * Route: a model with constraint rows runs from the workspace whenever one is given (more worlds
 * per CU than LDS allows, which hides the memory latency), and must have one when
 * mx_lds_bytes(model) > MX_LDS_BUDGET; otherwise, or with MX_FLAG_LDS, the working set is in LDS. */
size_t mx_workspace_bytes(const MxModel* model);

/* One control step for every world: `substeps` physics substeps (MX_FLAG_POLICY_FIRST marks the
 * first as the policy step).  Replaces Runtime.enqueue_action/enqueue_substep
 * (gpu/host/backends/cuda_fp32/runtime.py:40-77): step1 -> OSC -> solve -> integrate per substep.
 * Graph-capturable: no allocation, no host synchronisation. */
int mx_control_step(const MxModel* model, const MxData* data, int substeps, int flags, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  mx_control_step, with the
 * workspace slabs taken from a fixed device array of MX_SCRATCH_BYTES that the library holds per
 * device until the process ends, instead of data->workspace (ignored).  The call allocates nothing.
 * A batch whose slabs, (nworld + 1) * mx_workspace_bytes(model), exceed MX_SCRATCH_BYTES is refused
 * with MX_ERR_SCRATCH before any launch (models without constraint rows that fit LDS need none).
 * Every call on a device shares that device's array and leaves its contents behind; calls that
 * overlap on one device (other streams, other threads) race. */
int mx_control_step_noalloc(const MxModel* model, const MxData* data, int substeps, int flags, void* stream);

/* Forward pass (no integration) for the worlds whose mask entry is nonzero (mask may be null for
 * all worlds); with MX_FLAG_BOOTSTRAP also sets the OSC goal to the current end-effector pose.
 * Replaces Runtime.forward + Controller.bootstrap (gpu/host/backends/cuda_fp32/runtime.py:34-38,
 * controller.py:124-129). */
int mx_forward(const MxModel* model, const MxData* data, const int32_t* mask, int flags, void* stream);

/* mx_control_step with the observation plan sampled after every substep, inside the same launch
 * (qpos and qvel after the substep's integration, body and site poses before it, as the reference's
 * control graph samples after each substep: gpu/host/backends/cuda_fp32/runtime.py:47-56). */
int mx_control_step_observed(const MxModel* model, const MxData* data, const MxObsPlan* plan, int substeps,
                             int flags, void* stream);

/* One sampling call for the worlds whose mask entry is nonzero (all when mask is null), from the
 * published fields (the reference's forced sample after a reset, gpu/host/backends/cuda_fp32/
 * environment.py:211). */
int mx_observe(const MxModel* model, const MxData* data, const MxObsPlan* plan, const int32_t* mask, float dt,
               int force, void* stream);

/* Clear the plan's per-world state of the masked worlds: elapsed, present, cache, observed and sidequat
 * (sampled flags kept), as the reference's reset_observation (gpu/cuda/runtime/bridges.cu:172-178). */
int mx_observe_reset(const MxData* data, const MxObsPlan* plan, const int32_t* mask, void* stream);

size_t mx_obs_plan_bytes(void);              /* sizeof(MxObsPlan) */

/* The FP64 operational-space controller alone, for every world, from the controller inputs the last
 * control step published (osc_mass, osc_jac, osc_q, osc_qvel, osc_bias, osc_ee_pos/rot/vel): writes
 * osc_tau, ctrl of the OSC actuators, the gripper state, osc_error and osc_rank, and with
 * MX_FLAG_POLICY_FIRST first moves the goal by the action.  The reference's standalone controller
 * kernel (gpu/cuda/control/osc_solver.cu:309-727, ControllerSolveData), timed apart from the
 * physics for the heterogeneous benchmark batch. */
int mx_osc(const MxModel* model, const MxData* data, int flags, void* stream);

const char* mx_error_string(int code);

#ifdef __cplusplus
}
#endif
#endif /* MX_PHYSICS_H */
