"""GPU parity of the contact families and row kinds the benchmark scenes never produce.

The benchmark scenes rest every object on the table, give all geoms one material and no dof
friction, and send box-box pairs through GJK/EPA.  This scene covers the rest of the narrowphase and
row build, each compared with the CPU FP64 oracle from the same settled state by the same
one-substep comparison (and tolerances) as tests/test_gpu_contact_parity.py:

* on the ground plane: a box (plane_box), a capsule lying on its side (plane_capsule) and a sphere
  (plane_point);
* on the table: a sphere (sphere_box), a capsule (capsule_box), a hull (GJK/EPA) and two stacked
  boxes with a contact margin, which selects the primitive box-box routine (SAT and face clipping)
  for every box pair, the table included (gpu/host/backends/cuda_fp32/physics.py:90);
* unequal materials: friction, solref, solimp, solmix, priority and condim differ between objects
  (condim 1 frictionless rows next to condim 3 cones);
* dof friction-loss rows on two arm joints;
* the post-constraint stage on C3: cfrc_ext from contacts and applied body wrenches, cacc, cfrc_int,
  force and torque sensors at the grip site, gravity compensation (passive and actuator side).

Before comparing, each case counts the contacts per (geom type, geom type) family and the row kinds
and asserts that every family above occurred.
"""
import math

import numpy as np
import pytest

from libero_hip import scene as S
from test_gpu_contact_parity import _settled, compare_one_substep

pytestmark = pytest.mark.gpu

FAMILIES = {(S.PLANE, S.SPHERE): 'plane-sphere', (S.PLANE, S.CAPSULE): 'plane-capsule',
            (S.PLANE, S.BOX): 'plane-box', (S.SPHERE, S.BOX): 'sphere-box', (S.CAPSULE, S.BOX): 'capsule-box',
            (S.BOX, S.BOX): 'box-box (primitive)', (S.BOX, S.MESH): 'box-hull'}


def _sphere_body(rng, name, radius, **geom_kw):
    density = rng.uniform(500.0, 1500.0)
    mass = density * 4.0 / 3.0 * math.pi * radius ** 3
    b = S.Body(name, 0, mass=mass, inertia=(0.4 * mass * radius ** 2,) * 3)
    b.geoms.append(S.Geom(S.SPHERE, size=(radius, 0.0, 0.0), **geom_kw))
    b.joints.append(S.Joint(S.FREE))
    return b


def family_scene(nworld, seed=0, cone=S.PYRAMIDAL):
    rng = np.random.default_rng(seed)
    arm, actuators, osc, q_ready = S._arm()
    arm[1].joints[0].frictionloss = 0.3          # dof friction rows (link1, link2)
    arm[2].joints[0].frictionloss = 0.2
    bodies = [S._world(table=True)] + arm
    objects, slots = [], []

    def add(body, extent, xy, base):
        objects.append(body)
        slots.append((xy, base + extent))

    box, ext, _ = S._object(rng, 'box', 'floor_box')
    box.geoms[0].friction = (0.6, 0.005, 0.0001)
    add(box, ext, (1.2, -0.3), 0.0)
    cap, ext, _ = S._object(rng, 'capsule', 'floor_capsule')
    cap.geoms[0].solref = (0.03, 0.9)
    cap.geoms[0].solmix = 3.0
    add(cap, ext, (1.2, 0.0), 0.0)
    r = 0.03
    add(_sphere_body(rng, 'floor_ball', r, condim=1, priority=1), r, (1.3, 0.3), 0.0)
    r = 0.035
    add(_sphere_body(rng, 'table_ball', r, friction=(0.8, 0.005, 0.0001), solimp=(0.85, 0.97, 0.002, 0.4, 3.0)),
        r, (0.4, -0.25), S.TABLE_TOP)
    cap2, ext, _ = S._object(rng, 'capsule', 'table_capsule')
    cap2.geoms[0].friction = (1.3, 0.005, 0.0001)
    add(cap2, ext, (0.7, 0.25), S.TABLE_TOP)
    hull, ext, _ = S._object(rng, 'hull', 'table_hull')
    hull.geoms[0].solref = (0.015, 1.2)
    add(hull, ext, (0.45, 0.25), S.TABLE_TOP)
    lower, ext1, _ = S._object(rng, 'box', 'stack_lower')
    lower.geoms[0].margin = 0.002               # a box margin: primitive box-box for every box pair
    add(lower, ext1, (0.6, -0.05), S.TABLE_TOP)
    upper, ext2, _ = S._object(rng, 'box', 'stack_upper')
    upper.geoms[0].margin = 0.001
    upper.geoms[0].priority = 2
    upper.geoms[0].friction = (0.5, 0.005, 0.0001)
    add(upper, ext2, (0.6, -0.05), S.TABLE_TOP + 2 * ext1)
    bodies += objects
    opts = S.Options()
    opts.cone, opts.nconmax = cone, 64
    nq = 9 + 7 * len(objects)
    qpos = np.zeros((nworld, nq))
    for w in range(nworld):
        wrng = np.random.default_rng([seed, w])
        qpos[w, :7] = q_ready
        qpos[w, 7:9] = 0.02
        for k, ((x, y), z) in enumerate(slots):
            jitter = wrng.uniform(-0.01, 0.01, size=2) if k < len(slots) - 1 else 0.0
            q = S._qmul(S.quat_yaw(wrng.uniform(0, 2 * math.pi)), objects[k].quat)
            qpos[w, 9 + 7 * k:16 + 7 * k] = (x + (jitter[0] if k < len(slots) - 1 else 0.0),
                                             y + (jitter[1] if k < len(slots) - 1 else 0.0), z + 0.002, *q)
    return S.Scene(name='family', bodies=bodies, actuators=actuators, options=opts, nworld=nworld,
                   substeps=25, osc=osc, init_qpos=qpos, init_qvel=np.zeros((nworld, 9 + 6 * len(objects))),
                   seed=seed)


@pytest.mark.parametrize('cone,route', [('pyramidal', 'workspace'), ('pyramidal', 'lds'),
                                        ('elliptic', 'workspace'), ('elliptic', 'lds')])
def test_family_parity(gpu_available, cone, route):
    nworld = 24
    sc = family_scene(nworld, seed=7, cone=S.PYRAMIDAL if cone == 'pyramidal' else S.ELLIPTIC)
    m, dd, od, acts = _settled('family', nworld, settle=2, seed=7, scene=sc,
                               workspace=None if route == 'workspace' else False)
    assert m.boxbox_primitive == 1
    print('case family', cone, route, 'lds bytes', dd.dmodel.lds_bytes(), flush=True)
    families, rows = compare_one_substep(m, dd, od, acts[0], 'family %s %s' % (cone, route))
    print('families', {FAMILIES.get(k, k): v for k, v in sorted(families.items())}, 'row kinds', sorted(rows))
    for key, name in FAMILIES.items():
        assert families.get(key, 0) > 0, 'no %s contact occurred' % name
    assert 1 in rows                                      # dof friction-loss rows
    assert 5 in rows                                      # condim-1 frictionless rows
    assert (6 if cone == 'pyramidal' else 7) in rows


def post_scene(nworld, seed=0):
    """C3 with force / torque sensors at the grip site, gravity compensation on the arm (two joints
    reporting it as actuator force)."""
    sc = S.make_scene('c3', nworld, seed=seed)
    for k, body in enumerate(sc.bodies[2:10]):       # the seven links and the hand
        body.gravcomp = 0.6
        for j in body.joints:
            j.actuatorgravcomp = k in (1, 3)
    sc.sensors = [S.Sensor('force', 0), S.Sensor('torque', 0, cutoff=50.0)]
    return sc


@pytest.mark.parametrize('route', ['workspace', 'lds'])
def test_post_constraint_parity(gpu_available, route):
    """cfrc_ext (contacts and applied wrenches), cacc, cfrc_int, the force / torque sensors and
    gravity compensation against the oracle after one substep, 1e-4 relative per world."""
    import torch
    from helpers import rel_err
    from test_gpu_contact_parity import _np
    nworld = 32
    sc = post_scene(nworld, seed=5)
    m, dd, od, acts = _settled('post', nworld, settle=2, seed=5, scene=sc,
                               workspace=None if route == 'workspace' else False)
    assert m.nsensor == 2 and m.has_gravcomp
    rng = np.random.default_rng(6)
    xfrc = np.zeros((nworld, 6 * m.nbody))
    obj = m.nbody - 1                                # a hull pushed around in half of the worlds
    xfrc[::2, 6 * obj:6 * obj + 6] = rng.uniform(-0.5, 0.5, size=(nworld // 2, 6))
    od['xfrc_applied'][:] = xfrc
    dd['xfrc_applied'].copy_(torch.from_numpy(xfrc))
    print('case post', route, flush=True)
    compare_one_substep(m, dd, od, acts[0], 'post %s' % route)
    worst = {}
    for name in ('cfrc_ext', 'cfrc_int', 'cacc', 'sensordata', 'qfrc_passive', 'qfrc_actuator'):
        worst[name] = rel_err(_np(dd[name]), od[name], floor=1e-3)
    print('post', route, {k: '%.2e' % v for k, v in worst.items()})
    for k, v in worst.items():
        assert v < 1e-4, (k, v)
    assert np.abs(od['sensordata']).max() > 1.0 and np.abs(od['cfrc_ext']).max() > 1.0


@pytest.mark.parametrize('route', ['workspace', 'lds'])
def test_fluid_parity(gpu_available, route):
    """Inertia-box fluid forces (a dense, viscous medium with wind, so that they matter) on C3
    against the oracle after one substep: qfrc_passive and the step's outputs, 1e-4 relative."""
    from helpers import rel_err
    from test_gpu_contact_parity import _np
    nworld = 32
    sc = S.make_scene('c3', nworld, seed=3)
    sc.options.density, sc.options.viscosity, sc.options.wind = 300.0, 0.2, (0.5, -0.3, 0.0)
    m, dd, od, acts = _settled('fluid', nworld, settle=2, seed=3, scene=sc,
                               workspace=None if route == 'workspace' else False)
    assert m.has_fluid
    print('case fluid', route, flush=True)
    qvel0 = od['qvel'].copy()
    compare_one_substep(m, dd, od, acts[0], 'fluid %s' % route)
    err = rel_err(_np(dd['qfrc_passive']), od['qfrc_passive'], floor=1e-3)
    print('fluid', route, 'qfrc_passive %.2e' % err, 'max |qfrc_passive| %.3g' % np.abs(od['qfrc_passive']).max())
    assert err < 1e-4
    # the medium's share of the passive force is not negligible next to the joint dampers
    damper = -m.arrays['dof_damping'] * qvel0
    assert np.abs(od['qfrc_passive'] - damper).max() > 0.05 * np.abs(od['qfrc_passive']).max()
