"""Ordered low-dimensional observations sampled on the device, and their host packaging.

Mirrors the reference's observation contract:

* the plan schema (``ObservableSpec`` / ``ObservationPlan``, ``gpu/host/adapters/observations/schema.py:11-50``)
  and its default LIBERO plan (``plan_from_metadata``, ``schema.py:127-186``): robot joint positions,
  their cos / sin, joint velocities, end-effector position and quaternion, gripper joints, the
  inverse end-effector pose (inactive), and per object its position, quaternion and pose in the
  gripper frame;
* device sampling (``DeviceObservations``, ``gpu/host/backends/cuda_fp32/observations.py:19-110``):
  per-world clocks, values and presence in device arrays, sampled after every substep inside the
  control-step launch (``mx_control_step_observed``) or on demand (``mx_observe``, forced after a
  reset), reset per world (``mx_observe_reset``);
* host packaging at the action boundary (``pack_observations``, ``schema.py:99-125``): enabled and
  active observables in plan order plus the concatenated ``<modality>-state`` entries.

Quaternions follow robosuite (x, y, z, w).  The device library validates counts and pointers; this
module validates the plan's contents (offsets, indices, dependency order) before upload.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass
import ctypes as ct

import numpy as np

from . import native

OPS = {'gather': 0, 'cos': 1, 'sin': 2, 'inverse_pose': 3, 'relative_pos': 4, 'relative_quat': 5}
SOURCES = {'qpos': 0, 'qvel': 1, 'site_xpos': 2, 'body_xpos': 3, 'body_xquat': 4}
MAX_SPECS = 128


@dataclass(frozen=True)
class ObservableSpec:
    name: str
    modality: str
    operation: str          # qpos, qvel, site_pos, body_pos, body_quat, cos, sin, inverse_pose, relative_pos, relative_quat
    width: int
    indices: tuple = ()
    dependencies: tuple = ()
    period: float = 0.05
    enabled: bool = True
    active: bool = True
    shape: tuple = ()


@dataclass(frozen=True)
class ObservationPlan:
    specs: tuple
    order: tuple = ()

    @property
    def offsets(self):
        out, at = {}, 0
        for s in self.specs:
            out[s.name] = at
            at += s.width
        return out

    @property
    def width(self):
        return sum(s.width for s in self.specs)

    def validate(self):
        known = set()
        for s in self.specs:
            if s.name in known or s.width < 1 or not s.period > 0:
                raise ValueError('invalid observable descriptor: %s' % s.name)
            for name in s.dependencies:
                if name not in known:
                    raise ValueError('dependency %s must precede %s' % (name, s.name))
            known.add(s.name)
        if len(self.specs) > MAX_SPECS:
            raise ValueError('at most %d observables are sampled on the device' % MAX_SPECS)
        return self


def default_plan(model, *, prefix='robot0_', control_freq=None, use_object_obs=True):
    """The default LIBERO plan for a compiled model: the OSC arm, its two gripper joints, the
    end-effector site and body, and every free-jointed object body (period 1 / control_freq)."""
    a = model.arrays
    if control_freq is None:
        control_freq = 1.0 / (model.opt.timestep * model.scene.substeps)
    period = 1.0 / float(control_freq)
    specs, order = [], []

    def add(name, modality, op, width, indices=(), deps=(), active=True, shape=None):
        specs.append(ObservableSpec(name, modality, op, width, tuple(int(i) for i in indices), tuple(deps), period,
                                    True, active, (width,) if shape is None else shape))
        order.append(name)

    qa, da = a['osc_qposadr'], a['osc_dofadr']
    grip = [int(a['actuator_trnid'][k]) for k in a['osc_actuator'][7:9]]
    modality = prefix + 'proprio'
    add(prefix + 'joint_pos', modality, 'qpos', len(qa), qa)
    add(prefix + 'joint_pos_cos', modality, 'cos', len(qa), deps=(prefix + 'joint_pos',))
    add(prefix + 'joint_pos_sin', modality, 'sin', len(qa), deps=(prefix + 'joint_pos',))
    add(prefix + 'joint_vel', modality, 'qvel', len(da), da)
    add(prefix + 'eef_pos', modality, 'site_pos', 3, (model.osc_site,))
    add(prefix + 'eef_quat', modality, 'body_quat', 4, (int(a['site_body'][model.osc_site]),))
    add(prefix + 'gripper_qpos', modality, 'qpos', len(grip), [a['jnt_qposadr'][j] for j in grip])
    add(prefix + 'gripper_qvel', modality, 'qvel', len(grip), [a['jnt_dofadr'][j] for j in grip])
    if use_object_obs:
        add('world_pose_in_gripper', 'object', 'inverse_pose', 16, deps=(prefix + 'eef_pos', prefix + 'eef_quat'),
            active=False, shape=(4, 4))
        for b, body in enumerate(model.scene.bodies):
            if b == 0 or model.scene.bodies[body.parent] is not model.scene.bodies[0] or not body.joints \
                    or body.joints[0].type != 0:
                continue
            name = body.name
            add(name + '_pos', 'object', 'body_pos', 3, (b,))
            add(name + '_quat', 'object', 'body_quat', 4, (b,))
            rel = name + '_to_' + prefix + 'eef_pos'
            add(rel, 'object', 'relative_pos', 3, deps=(name + '_pos', name + '_quat', 'world_pose_in_gripper'))
            add(name + '_to_' + prefix + 'eef_quat', 'object', 'relative_quat', 4, deps=(rel,))
    return ObservationPlan(tuple(specs), tuple(order)).validate()


def plan_metadata(plan, model):
    """The device arrays of a plan (int32 / float32 numpy): op, offset, size, index_offset, indices,
    dep0..2, presence, enabled, period.  Gather indices are MX_OBS_SRC << 24 | element."""
    offsets = plan.offsets
    ids = {s.name: i for i, s in enumerate(plan.specs)}
    widths = dict(qpos=model.nq, qvel=model.nv, site_xpos=3 * model.nsite, body_xpos=3 * model.nbody,
                  body_xquat=4 * model.nbody)
    op, off, size, ixoff, ix, d0, d1, d2, pres, en, per = ([] for _ in range(11))
    for s in plan.specs:
        ixoff.append(len(ix))
        deps = [offsets[d] for d in s.dependencies]
        if s.operation in ('qpos', 'qvel', 'site_pos', 'body_pos', 'body_quat'):
            source = {'site_pos': 'site_xpos', 'body_pos': 'body_xpos', 'body_quat': 'body_xquat'}.get(s.operation,
                                                                                                   s.operation)
            if s.operation == 'body_quat':            # MuJoCo w x y z -> robosuite x y z w
                local = [4 * s.indices[0] + j for j in (1, 2, 3, 0)]
            elif s.operation in ('site_pos', 'body_pos'):
                local = [3 * s.indices[0] + j for j in range(3)]
            else:
                local = list(s.indices)
            if len(local) != s.width or any(i < 0 or i >= widths[source] for i in local):
                raise ValueError('source index out of range: %s' % s.name)
            ix.extend((SOURCES[source] << 24) | int(i) for i in local)
            op.append(OPS['gather'])
        elif s.operation in OPS:
            op.append(OPS[s.operation])
        else:
            raise NotImplementedError(s.operation)
        need = {'cos': 1, 'sin': 1, 'inverse_pose': 2, 'relative_pos': 3, 'relative_quat': 1}.get(s.operation, 0)
        if len(s.dependencies) != need:
            raise ValueError('%s takes %d dependencies' % (s.name, need))
        deps += [0] * (3 - len(deps))
        d0.append(deps[0]); d1.append(deps[1]); d2.append(deps[2])
        pres.extend([ids[d] for d in s.dependencies] + [-1] * (3 - len(s.dependencies)))
        off.append(offsets[s.name]); size.append(s.width); en.append(int(s.enabled)); per.append(s.period)
    i32 = lambda x: np.asarray(x if len(x) else [0], np.int32)   # noqa: E731
    return dict(op=i32(op), offset=i32(off), size=i32(size), index_offset=i32(ixoff), indices=i32(ix), dep0=i32(d0),
                dep1=i32(d1), dep2=i32(d2), presence=i32(pres), enabled=i32(en),
                period=np.asarray(per, np.float32))


def pack_observations(plan, values):
    """One world's observed values at an action boundary: enabled and active observables in plan
    order, then the concatenated ``<modality>-state`` groups (reference schema.py:99-125)."""
    values = np.asarray(values)
    if values.shape != (plan.width,):
        raise ValueError('observed buffer shape %s, expected %s' % (values.shape, (plan.width,)))
    offsets = plan.offsets
    result, groups = OrderedDict(), OrderedDict()
    for s in plan.specs:
        if s.enabled and s.active:
            data = values[offsets[s.name]:offsets[s.name] + s.width].copy()
            value = data[0] if s.shape == (1,) else data.reshape(s.shape or ())
            result[s.name] = value
            groups.setdefault(s.modality + '-state', []).append(np.atleast_1d(value))
    if plan.order:
        result = OrderedDict((n, result[n]) for n in plan.order if n in result)
    for modality, group in groups.items():
        result[modality] = np.concatenate(group, axis=-1)
    return result


class DeviceObservations:
    """A plan's metadata and per-world sampling state in device tensors, bound to MxObsPlan."""

    def __init__(self, plan, model, nworld, device='cuda:0'):
        import torch
        self.plan = plan.validate()
        self.model = model
        self.nworld = nworld
        self.device = torch.device(device)
        meta = plan_metadata(plan, model)
        self.meta = {k: torch.from_numpy(v).to(self.device) for k, v in meta.items()}
        ns, width = len(plan.specs), plan.width
        f32 = lambda *s: torch.zeros(s, dtype=torch.float32, device=self.device)   # noqa: E731
        i32 = lambda *s: torch.zeros(s, dtype=torch.int32, device=self.device)     # noqa: E731
        self.state = dict(cache=f32(nworld, width), observed=f32(nworld, width), sidequat=f32(nworld, width),
                          elapsed=f32(nworld, ns), sampled=i32(nworld, ns), present=i32(nworld, ns),
                          events=i32(nworld, ns))
        s = native.MxObsPlan()
        s.nspec, s.width = ns, width
        for name, t in list(self.meta.items()) + list(self.state.items()):
            ctype = ct.c_float if t.dtype == torch.float32 else ct.c_int32
            setattr(s, name, ct.cast(ct.c_void_p(t.data_ptr()), ct.POINTER(ctype)))
        self.struct = s

    @property
    def observed(self):
        return self.state['observed']

    def control_step(self, data, substeps, flags=native.FLAG_POLICY_FIRST, stream=None):
        rc = native.load().mx_control_step_observed(ct.byref(data.dmodel.struct), ct.byref(data.struct),
                                                    ct.byref(self.struct), substeps, flags, data._stream(stream))
        native.check(rc, 'mx_control_step_observed')

    def sample(self, data, mask=None, dt=None, force=False, stream=None):
        dt = self.model.opt.timestep if dt is None else dt
        ptr = None if mask is None else ct.c_void_p(mask.data_ptr())
        rc = native.load().mx_observe(ct.byref(data.dmodel.struct), ct.byref(data.struct), ct.byref(self.struct),
                                      ptr, float(dt), int(force), data._stream(stream))
        native.check(rc, 'mx_observe')

    def reset(self, data, mask=None, stream=None):
        ptr = None if mask is None else ct.c_void_p(mask.data_ptr())
        rc = native.load().mx_observe_reset(ct.byref(data.struct), ct.byref(self.struct), ptr, data._stream(stream))
        native.check(rc, 'mx_observe_reset')

    def pack(self, values_row):
        return pack_observations(self.plan, values_row)
