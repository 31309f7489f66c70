"""Field tables of the C ABI (include/mx_physics.h) and the packing of a compiled model.

The tables below list the X-macro fields of ``MxModel`` / ``MxData`` in declaration order; the
loader compares them with the names the library exports (``mx_field_name``), the same ABI check
the reference performs with ``flash_<leaf>_arguments_bytes`` (``gpu/host/runtime/dynamics/mjwarp_motion.py:20-37``).
Per-world arrays are world-major, ``(nworld, width)``.
"""
from __future__ import annotations

import ctypes as ct
import numpy as np

ABI_VERSION = 18
LDS_BUDGET = 163840          # MX_LDS_BUDGET: LDS of one gfx950 workgroup

MODEL_REAL_ARRAYS = [
    'body_pos', 'body_quat', 'body_ipos', 'body_iquat', 'body_mass', 'body_subtreemass',
    'body_inertia', 'body_invweight0',
    'jnt_pos', 'jnt_axis', 'jnt_range', 'jnt_stiffness', 'jnt_margin', 'jnt_solref', 'jnt_solimp',
    'qpos0', 'qpos_spring',
    'dof_armature', 'dof_damping', 'dof_frictionloss', 'dof_invweight0', 'dof_solref', 'dof_solimp',
    'geom_pos', 'geom_quat', 'geom_size', 'geom_rbound', 'geom_aabb', 'geom_friction',
    'geom_solref', 'geom_solimp', 'geom_solmix', 'geom_margin', 'geom_gap',
    'site_pos', 'site_quat', 'mesh_vert', 'mesh_polynormal',
    'actuator_gear', 'actuator_gainprm', 'actuator_biasprm', 'actuator_ctrlrange', 'actuator_forcerange',
    'body_gravcomp', 'sensor_cutoff']

MODEL_INT_ARRAYS = [
    'body_parent', 'body_rootid', 'body_weldid', 'body_treeid', 'body_jntadr', 'body_jntnum',
    'body_dofadr', 'body_dofnum', 'body_subtreesize', 'body_lastdof', 'level_adr', 'level_body',
    'jnt_type', 'jnt_body', 'jnt_qposadr', 'jnt_dofadr', 'jnt_limited',
    'dof_body', 'dof_jnt', 'dof_parent', 'dof_treeid',
    'tree_dofadr', 'tree_dofnum', 'tree_madr', 'tree_dampadr', 'mpair_i', 'mpair_j',
    'geom_type', 'geom_body', 'geom_contype', 'geom_conaffinity', 'geom_condim', 'geom_priority',
    'geom_dataid', 'site_body', 'mesh_vertadr', 'mesh_vertnum',
    'mesh_polynum', 'mesh_polyadr', 'mesh_polyvertadr', 'mesh_polyvertnum', 'mesh_polyvert',
    'mesh_polymapadr', 'mesh_polymapnum', 'mesh_polymap',
    'actuator_trnid', 'actuator_biastype', 'actuator_ctrllimited', 'actuator_forcelimited',
    'pair_geom', 'osc_qposadr', 'osc_dofadr', 'osc_actuator',
    'jnt_actgravcomp', 'sensor_type', 'sensor_objid', 'sensor_adr', 'sensor_datatype']

MODEL_INT_SCALARS = [
    'abi_version', 'nq', 'nv', 'nu', 'nbody', 'njnt', 'ngeom', 'nsite', 'nmesh', 'nmeshvert',
    'npair', 'ntree', 'nM', 'nMpair', 'nlevel', 'nconmax', 'njmax',
    'opt_iterations', 'opt_ls_iterations', 'opt_cone', 'opt_disableflags',
    'osc_site', 'osc_uncouple', 'has_body_active', 'maxchain', 'maxtree', 'maxpairdof',
    'opt_ccd_iterations', 'epa_iterations', 'boxbox_primitive',
    'nsensor', 'nsensordata', 'has_gravcomp', 'has_fluid', 'nMdamp', 'osc_ndof', 'convex_mpr',
    'opt_mpr_iterations', 'osc_action_scaled']

MODEL_REAL_SCALARS = [
    'opt_timestep', 'opt_tolerance', 'opt_ls_tolerance', 'opt_impratio',
    'opt_gravity_x', 'opt_gravity_y', 'opt_gravity_z', 'osc_gripper_speed', 'meaninertia',
    'opt_ccd_tolerance', 'opt_density', 'opt_viscosity', 'opt_wind_x', 'opt_wind_y', 'opt_wind_z',
    'opt_mpr_tolerance']

DATA_REAL_ARRAYS = [
    'time', 'qpos', 'qvel', 'ctrl', 'qacc_warmstart', 'qfrc_applied',
    'qacc', 'qacc_smooth', 'qfrc_bias', 'qfrc_passive', 'qfrc_actuator', 'qfrc_smooth',
    'qfrc_constraint', 'actuator_force', 'M',
    'xpos', 'xquat', 'xmat', 'geom_xpos', 'geom_xmat', 'site_xpos', 'site_xmat', 'subtree_com',
    'osc_mass', 'osc_jac', 'osc_q', 'osc_qvel', 'osc_bias', 'osc_ee_pos', 'osc_ee_rot', 'osc_ee_vel',
    'contact_pos', 'contact_frame', 'contact_dist', 'contact_friction', 'contact_includemargin',
    'efc_force', 'efc_pos', 'efc_D', 'efc_aref',
    'xfrc_applied', 'cacc', 'cfrc_int', 'cfrc_ext', 'sensordata']

DATA_F64_ARRAYS = ['osc_action', 'osc_goal_pos', 'osc_goal_rot', 'osc_gripper', 'osc_gains', 'osc_q0', 'osc_tau',
                   'osc_action_scale', 'stat_sums', 'workspace']

DATA_INT_ARRAYS = ['overflow', 'osc_error', 'osc_rank', 'nstep', 'body_active',
                   'ncon', 'contact_geom', 'contact_dim', 'nefc', 'efc_type', 'efc_state', 'efc_id', 'solver_niter']

TABLES = [MODEL_REAL_ARRAYS, MODEL_INT_ARRAYS, MODEL_INT_SCALARS, MODEL_REAL_SCALARS,
          DATA_REAL_ARRAYS, DATA_F64_ARRAYS, DATA_INT_ARRAYS]


def data_widths(m, workspace_doubles=0):
    """Per-world width of every data array for compiled model ``m`` (``workspace`` is sized by the
    library, ``mx_workspace_bytes``; 0 when the working set stays in LDS)."""
    nq, nv, nu, nb = m.nq, m.nv, m.nu, m.nbody
    on = m.osc_ndof          # arm joints of the controller
    w = dict(time=1, qpos=nq, qvel=nv, ctrl=nu, qacc_warmstart=nv, qfrc_applied=nv, qacc=nv,
             qacc_smooth=nv, qfrc_bias=nv, qfrc_passive=nv, qfrc_actuator=nv, qfrc_smooth=nv,
             qfrc_constraint=nv, actuator_force=nu, M=m.nM, xpos=3 * nb, xquat=4 * nb, xmat=9 * nb,
             geom_xpos=3 * m.ngeom, geom_xmat=9 * m.ngeom, site_xpos=3 * m.nsite, site_xmat=9 * m.nsite,
             subtree_com=3 * nb, osc_mass=on * on, osc_jac=6 * on, osc_q=on, osc_qvel=on, osc_bias=on,
             osc_ee_pos=3, osc_ee_rot=9, osc_ee_vel=6,
             osc_action=7, osc_goal_pos=3, osc_goal_rot=9, osc_gripper=2, osc_gains=12, osc_q0=on,
             osc_tau=on, osc_action_scale=24, stat_sums=4, overflow=1, osc_error=1, osc_rank=3, nstep=1, body_active=nb,
             workspace=workspace_doubles, xfrc_applied=6 * nb, cacc=6 * nb, cfrc_int=6 * nb, cfrc_ext=6 * nb,
             sensordata=max(m.nsensordata, 1))
    C, R = max(m.nconmax, 1), max(m.njmax, 1)
    w.update(contact_pos=3 * C, contact_frame=9 * C, contact_dist=C, contact_friction=5 * C,
             contact_includemargin=C, efc_force=R, efc_pos=R, efc_D=R, efc_aref=R, ncon=1,
             contact_geom=2 * C, contact_dim=C, nefc=1, efc_type=R, efc_state=R, efc_id=R, solver_niter=1)
    return w


def model_scalars(m):
    o = m.opt
    return dict(abi_version=ABI_VERSION, nq=m.nq, nv=m.nv, nu=m.nu, nbody=m.nbody, njnt=m.njnt,
                ngeom=m.ngeom, nsite=m.nsite, nmesh=m.nmesh, nmeshvert=m.nmeshvert, npair=m.npair,
                ntree=m.ntree, nM=m.nM, nMpair=m.nMpair, nlevel=m.nlevel, nconmax=m.nconmax,
                njmax=m.njmax, opt_iterations=o.iterations, opt_ls_iterations=o.ls_iterations,
                opt_cone=o.cone, opt_disableflags=o.disableflags, osc_site=m.osc_site,
                osc_uncouple=m.osc_uncouple, has_body_active=int(m.body_active is not None),
                maxchain=m.maxchain, maxtree=m.maxtree, maxpairdof=m.maxpairdof,
                opt_ccd_iterations=o.ccd_iterations, epa_iterations=m.epa_iterations,
                boxbox_primitive=m.boxbox_primitive, opt_ccd_tolerance=o.ccd_tolerance,
                nsensor=m.nsensor, nsensordata=m.nsensordata, has_gravcomp=m.has_gravcomp,
                has_fluid=m.has_fluid, nMdamp=m.nMdamp, osc_ndof=m.osc_ndof, convex_mpr=m.convex_mpr,
                opt_mpr_iterations=o.mpr_iterations, osc_action_scaled=m.osc_action_scaled, opt_mpr_tolerance=o.mpr_tolerance, opt_density=o.density, opt_viscosity=o.viscosity,
                opt_wind_x=o.wind[0], opt_wind_y=o.wind[1], opt_wind_z=o.wind[2],
                opt_timestep=o.timestep, opt_tolerance=o.tolerance, opt_ls_tolerance=o.ls_tolerance,
                opt_impratio=o.impratio, opt_gravity_x=o.gravity[0], opt_gravity_y=o.gravity[1],
                opt_gravity_z=o.gravity[2], osc_gripper_speed=m.osc_gripper_speed,
                meaninertia=m.meaninertia)


def model_arrays(m):
    """Flattened model arrays (real ones in float64, int ones in int32), in ABI order."""
    a = m.arrays
    real = {name: np.ascontiguousarray(np.asarray(a[name], np.float64).reshape(-1)) for name in MODEL_REAL_ARRAYS}
    ints = {name: np.ascontiguousarray(np.asarray(a[name], np.int32).reshape(-1)) for name in MODEL_INT_ARRAYS}
    return real, ints


def make_struct(name, real_ctype, scalar_real_ctype, kind):
    """ctypes mirror of MxModel (kind='model') or MxData (kind='data')."""
    fields = []
    if kind == 'model':
        fields += [(n, ct.c_int32) for n in MODEL_INT_SCALARS]
        fields += [(n, scalar_real_ctype) for n in MODEL_REAL_SCALARS]
        fields += [(n, ct.POINTER(real_ctype)) for n in MODEL_REAL_ARRAYS]
        fields += [(n, ct.POINTER(ct.c_int32)) for n in MODEL_INT_ARRAYS]
    else:
        fields += [('nworld', ct.c_int32), ('workspace_doubles', ct.c_int32), ('workspace_total', ct.c_int64)]
        fields += [(n, ct.POINTER(real_ctype)) for n in DATA_REAL_ARRAYS]
        fields += [(n, ct.POINTER(ct.c_double)) for n in DATA_F64_ARRAYS]
        fields += [(n, ct.POINTER(ct.c_int32)) for n in DATA_INT_ARRAYS]
    return type(name, (ct.Structure,), {'_fields_': fields})


def check_field_tables(count_fn, name_fn, label):
    """Compare the Python tables with the names exported by a loaded library."""
    for which, table in enumerate(TABLES):
        n = count_fn(which)
        names = [name_fn(which, i).decode() for i in range(n)]
        if names != table:
            raise ImportError('%s ABI field table %d differs: %s != %s' % (label, which, names, table))


def pack_arena(arrays, dtype):
    """Concatenate named 1-D arrays into one aligned arena; returns (arena, {name: offset})."""
    offsets, total = {}, 0
    itemsize = np.dtype(dtype).itemsize
    align = max(1, 64 // itemsize)
    for name, arr in arrays.items():
        offsets[name] = total
        total += (len(arr) + align - 1) // align * align
    arena = np.zeros(max(total, align), dtype)
    for name, arr in arrays.items():
        arena[offsets[name]:offsets[name] + len(arr)] = arr
    return arena, offsets
