"""Pins of the oracle's gravity compensation, applied body wrenches, post-constraint forces and
force / torque sensors by Newton-Euler balance (no code shared with the oracle).

The oracle restates the reference's rigid_gravity_projection (gpu/cuda/dynamics/mjwarp_queries.cu:55),
cfrc_ext (mjwarp_external_wrench.cu:26-90), world_postconstraint (mjwarp_postconstraint.cu:87) and
force_torque_sensors (mjwarp_queries.cu:31).  Checks:

* gravity compensation 1 on every arm body holds the arm still (qacc = 0 at rest); compensation c
  gives the accelerations of gravity scaled by 1 - c; reported as actuator force it moves from
  qfrc_passive to qfrc_actuator without changing qacc;
* an applied wrench equal to a free body's weight cancels gravity; an applied torque gives the
  angular acceleration I^-1 tau (body frame, at rest);
* a free body's joint transmits nothing: cfrc_int of a free root body is zero (its inertial forces
  balance gravity and cfrc_ext), for bodies resting on, sliding over or falling onto the plane;
* a box at rest on the plane: cfrc_ext carries its weight and no torque about its centre of mass;
* force and torque sensors at the grip site of a static arm read the weight of the hand's subtree and
  its moment about the site, in the site frame (closed forms from the bodies' masses and centres).
"""
import numpy as np
import pytest

from libero_hip import native, scene as S
from libero_hip.model import Model
from helpers import make_oracle
from test_oracle_constraint_pins import _scene, _oracle, _sphere

G = 9.81


def _arm_scene(gravcomp=0.0, actuatorgravcomp=False, sensors=(), gravity=(0.0, 0.0, -G)):
    sc = _scene([], np.zeros(0), gravity=gravity)
    for body in sc.bodies[1:]:
        body.gravcomp = gravcomp
        for j in body.joints:
            j.actuatorgravcomp = actuatorgravcomp
    sc.sensors = [S.Sensor(kind, 0) for kind in sensors]
    return sc


def _rest(od):
    od['qvel'][:] = 0
    od['ctrl'][:] = 0
    od['ctrl'][:, 7:9] = od['qpos'][:, 7:9]      # finger servos at their current positions
    od.forward(None, native.FLAG_NO_CONTROL)


def test_full_gravity_compensation_holds_the_arm():
    m, om, od = _oracle(_arm_scene(gravcomp=1.0))
    _rest(od)
    assert np.abs(od['qacc'][0, :9]).max() < 1e-10
    assert np.abs(od['qfrc_passive'][0, :9]).max() > 1.0          # the compensation is there


@pytest.mark.parametrize('c', [0.25, 0.5, 0.9])
def test_partial_compensation_scales_gravity(c):
    m, om, od = _oracle(_arm_scene(gravcomp=c))
    _rest(od)
    m2, om2, od2 = _oracle(_arm_scene(gravity=(0.0, 0.0, -G * (1 - c))))
    _rest(od2)
    np.testing.assert_allclose(od['qacc'][0, :9], od2['qacc'][0, :9], rtol=1e-9, atol=1e-10)


def test_compensation_reported_as_actuator_force():
    m, om, od = _oracle(_arm_scene(gravcomp=0.7))
    _rest(od)
    m2, om2, od2 = _oracle(_arm_scene(gravcomp=0.7, actuatorgravcomp=True))
    _rest(od2)
    np.testing.assert_allclose(od['qacc'], od2['qacc'], rtol=1e-12, atol=1e-12)
    moved = od['qfrc_passive'] - od2['qfrc_passive']
    np.testing.assert_allclose(od2['qfrc_actuator'] - od['qfrc_actuator'], moved, rtol=1e-12, atol=1e-12)
    assert np.abs(moved).max() > 1.0


def _floating_box():
    half = (0.03, 0.04, 0.05)
    mass = 0.8
    body = S.Body('box', 0, mass=mass, inertia=S.box_inertia(mass, half))
    body.geoms.append(S.Geom(S.BOX, size=half))
    body.joints.append(S.Joint(S.FREE))
    return body, mass


def test_applied_weight_cancels_gravity_and_torque_spins():
    body, mass = _floating_box()
    q = np.array([0.9, 0.1, -0.3, 0.2])
    q /= np.linalg.norm(q)
    sc = _scene([body], [[0.3, 0.4, 1.5, *q]])
    m, om, od = _oracle(sc)
    b = m.nbody - 1
    tau = np.array([0.3, -0.2, 0.5])
    od['xfrc_applied'][0, 6 * b:6 * b + 6] = [0.0, 0.0, mass * G, *tau]
    od.forward(None, native.FLAG_NO_CONTROL)
    qacc = od['qacc'][0, 9:15]
    assert np.abs(qacc[:3]).max() < 1e-12                          # weight cancelled
    R = od['xmat'][0, 9 * b:9 * b + 9].reshape(3, 3)
    inertia = np.array(S.box_inertia(mass, (0.03, 0.04, 0.05)))
    np.testing.assert_allclose(qacc[3:], (R.T @ tau) / inertia, rtol=1e-10)   # body-frame rotation dofs
    # the applied wrench is part of cfrc_ext, about the body's centre of mass (its own root)
    np.testing.assert_allclose(od['cfrc_ext'][0, 6 * b:6 * b + 6], [*tau, 0.0, 0.0, mass * G], atol=1e-12)


@pytest.mark.parametrize('cone', [S.PYRAMIDAL, S.ELLIPTIC])
def test_free_bodies_transmit_nothing_through_their_joint(cone):
    """cfrc_int of a free root body vanishes: resting, sliding and falling boxes and spheres."""
    body, mass = _floating_box()
    ball = _sphere(0.5, 0.04, condim=3)
    sc = _scene([body, ball], [[0.3, 0.4, 0.049, 1.0, 0.0, 0.0, 0.0, 0.6, -0.2, 0.03, 1.0, 0.0, 0.0, 0.0]],
                cone=cone, nworld=3)
    sc.init_qpos[1, 9:12] = (0.3, 0.4, 0.3)         # box above the floor: no contact
    m, om, od = _oracle(sc)
    od['qvel'][2, 9:12] = (0.4, -0.1, 0.0)           # world 2: sliding box
    od['qvel'][2, 15:18] = (0.0, 0.3, 0.2)
    for _ in range(3):
        od.control_step(5, native.FLAG_NO_CONTROL)
    roots = [m.nbody - 2, m.nbody - 1]
    assert (od["ncon"][[0, 2], 0] >= 2).all()
    for w in range(3):
        for b in roots:
            f = od['cfrc_int'][w, 6 * b:6 * b + 6]
            scale = 0.8 * G
            assert np.abs(f).max() < 1e-9 * scale, (w, b, f)


@pytest.mark.parametrize('cone', [S.PYRAMIDAL, S.ELLIPTIC])
def test_resting_box_contacts_carry_its_weight(cone):
    body, mass = _floating_box()
    sc = _scene([body], [[0.3, 0.4, 0.05, 1.0, 0.0, 0.0, 0.0]], cone=cone)
    m, om, od = _oracle(sc)
    for _ in range(20):
        od.control_step(25, native.FLAG_NO_CONTROL)
    b = m.nbody - 1
    ext = od['cfrc_ext'][0, 6 * b:6 * b + 6]
    np.testing.assert_allclose(ext[3:], [0.0, 0.0, mass * G], atol=1e-5 * mass * G)
    assert np.abs(ext[:3]).max() < 1e-5 * mass * G * 0.05      # no torque about the centre of mass


def test_static_arm_force_torque_sensors():
    sc = _arm_scene(gravcomp=1.0, sensors=('force', 'torque'))
    m, om, od = _oracle(sc)
    rng = np.random.default_rng(3)
    od['qpos'][0, :7] += rng.uniform(-0.4, 0.4, 7)
    _rest(od)
    assert np.abs(od['qacc'][0, :9]).max() < 1e-9                 # static
    a = m.arrays
    site = 0
    hand = int(a['site_body'][site])
    sub = range(hand, hand + int(a['body_subtreesize'][hand]))
    masses = a['body_mass'][list(sub)]
    xipos = np.array([od['xpos'][0, 3 * k:3 * k + 3] + od['xmat'][0, 9 * k:9 * k + 9].reshape(3, 3)
                      @ a['body_ipos'][k] for k in sub])
    s_pos = od['site_xpos'][0, :3]
    R = od['site_xmat'][0, :9].reshape(3, 3)
    weight = np.array([0.0, 0.0, masses.sum() * G])
    moment = sum(np.cross(x - s_pos, [0.0, 0.0, mk * G]) for x, mk in zip(xipos, masses))
    np.testing.assert_allclose(od['sensordata'][0, :3], R.T @ weight, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(od['sensordata'][0, 3:6], R.T @ moment, rtol=1e-9, atol=1e-12)
    # cutoff clips each value to [-cutoff, cutoff]
    sc.sensors[0].cutoff = 1.0
    m2, om2, od2 = _oracle(sc)
    od2['qpos'][:] = od['qpos']
    _rest(od2)
    np.testing.assert_allclose(od2['sensordata'][0, :3], np.clip(R.T @ weight, -1.0, 1.0), rtol=1e-9, atol=1e-12)
