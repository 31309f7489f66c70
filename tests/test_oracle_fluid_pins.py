"""Pins of the oracle's inertia-box fluid forces (MuJoCo's mj_inertiaBoxFluidModel, restated from the
reference's gpu/cuda/fp32/fused_motion_passive.cu:253-330) by data the oracle does not compute:

* a free box: the equivalent box of its inertia is the box itself, so the drag on a translating or
  spinning box follows from its geom half-sizes alone (closed forms in the box frame, wind included);
  the translational dofs carry the world-frame force, the rotational dofs the body-frame torque;
* an articulated arm in random motion: every body's centre-of-mass velocity and angular velocity by
  central differences of forward kinematics, and the fluid's generalized force must do exactly the
  power the drag law gives on those velocities (negative: the medium only dissipates);
* density or viscosity zero switches the corresponding terms off, and the passive-force switch
  switches all of them off.
"""
import numpy as np
import pytest

from libero_hip import native, scene as S
from libero_hip.model import quat2mat
from test_oracle_constraint_pins import _scene, _oracle

RHO, MU = 40.0, 0.3


def _medium(sc, density=RHO, viscosity=MU, wind=(0.0, 0.0, 0.0)):
    sc.options.density, sc.options.viscosity, sc.options.wind = density, viscosity, wind
    sc.options.gravity = (0.0, 0.0, 0.0)
    return sc


def _box(half, mass=0.9):
    body = S.Body('box', 0, mass=mass, inertia=S.box_inertia(mass, half))
    body.geoms.append(S.Geom(S.BOX, size=half))
    body.joints.append(S.Joint(S.FREE))
    return body


def _drag(s, v, w, rho, mu):
    """Force and torque of the drag law on a box of full sides s, in its own frame."""
    d = s.mean()
    f = -3 * np.pi * mu * d * v
    t = -np.pi * mu * d ** 3 * w
    for k in range(3):
        i, j = [a for a in range(3) if a != k]
        f[k] -= 0.5 * rho * s[i] * s[j] * abs(v[k]) * v[k]
        t[k] -= rho / 64 * s[k] * (s[i] ** 4 + s[j] ** 4) * abs(w[k]) * w[k]
    return f, t


def _fluid_force(sc_factory, qpos, qvel, **medium):
    """qfrc_passive with the medium minus without it (joint dampers and springs cancel)."""
    out = []
    for kw in (medium, dict(density=0.0, viscosity=0.0)):
        m, om, od = _oracle(_medium(sc_factory(), **kw))
        od['qpos'][:] = qpos
        od['qvel'][:] = qvel
        od['ctrl'][:] = 0
        od.forward(None, native.FLAG_NO_CONTROL)
        out.append(od['qfrc_passive'][0].copy())
    return out[0] - out[1], m, od


@pytest.mark.parametrize('wind', [(0.0, 0.0, 0.0), (0.7, -0.4, 0.2)])
@pytest.mark.parametrize('density,viscosity', [(RHO, MU), (RHO, 0.0), (0.0, MU)])
def test_free_box_drag_closed_form(density, viscosity, wind):
    half = np.array([0.03, 0.05, 0.08])
    q = np.array([0.8, 0.3, -0.4, 0.2])
    q /= np.linalg.norm(q)
    qpos = np.r_[np.zeros(9), 0.3, 0.2, 1.0, q]
    qpos[7:9] = 0.02
    rng = np.random.default_rng(11)
    for _ in range(4):
        qvel = np.r_[np.zeros(9), rng.uniform(-2, 2, 3), rng.uniform(-6, 6, 3)]
        f, m, od = _fluid_force(lambda: _scene([_box(tuple(half))], qpos[9:]), qpos, qvel,
                                density=density, viscosity=viscosity, wind=wind)
        R = quat2mat(q)
        v_local = R.T @ (qvel[9:12] - np.array(wind))
        fl, tl = _drag(2 * half, v_local, qvel[12:15], density, viscosity)
        scale = max(np.abs(fl).max(), np.abs(tl).max())
        assert scale > 1e-3
        np.testing.assert_allclose(f[9:12], R @ fl, rtol=1e-10, atol=1e-12 * scale)
        np.testing.assert_allclose(f[12:15], tl, rtol=1e-10, atol=1e-12 * scale)
        if not any(wind):
            assert np.abs(f[:9]).max() == 0.0              # the parked arm is at rest in still air


def _body_velocities(sc_factory, qpos, qvel, eps=1e-6):
    """Centre-of-mass and angular velocities of every body by central differences (hinge/slide)."""
    frames = []
    for sign in (1, -1):
        m, om, od = _oracle(_medium(sc_factory(), density=0.0, viscosity=0.0))
        od['qpos'][:] = qpos + sign * eps * qvel
        od['qvel'][:] = 0
        od.forward(None, native.FLAG_NO_CONTROL)
        a = m.arrays
        xi, Ri = [], []
        for b in range(m.nbody):
            R = od['xmat'][0, 9 * b:9 * b + 9].reshape(3, 3)
            xi.append(od['xpos'][0, 3 * b:3 * b + 3] + R @ a['body_ipos'][b])
            Ri.append(R @ quat2mat(a['body_iquat'][b]))
        frames.append((np.array(xi), np.array(Ri)))
    (xp, Rp), (xm, Rm) = frames
    v = (xp - xm) / (2 * eps)
    R0 = (Rp + Rm) / 2
    W = np.einsum('bij,bkj->bik', (Rp - Rm) / (2 * eps), R0)   # Rdot R^T = [w]x (world)
    w = np.stack([W[:, 2, 1], W[:, 0, 2], W[:, 1, 0]], axis=1)
    return v, w, R0


def test_arm_fluid_power_matches_the_drag_law():
    rng = np.random.default_rng(4)
    factory = lambda: _scene([], np.zeros(0))
    for trial in range(5):
        m0, om0, od0 = _oracle(factory())
        qpos = od0['qpos'][0].copy()
        qpos[:7] += rng.uniform(-0.6, 0.6, 7)
        qvel = rng.uniform(-2.0, 2.0, m0.nv)
        f, m, od = _fluid_force(factory, qpos, qvel)
        v, w, R = _body_velocities(factory, qpos, qvel)
        a = m.arrays
        power = 0.0
        for b in range(1, m.nbody):
            mass, inertia = a['body_mass'][b], a['body_inertia'][b]
            s = np.sqrt(np.maximum(1e-15, [inertia[1] + inertia[2] - inertia[0],
                                           inertia[0] + inertia[2] - inertia[1],
                                           inertia[0] + inertia[1] - inertia[2]]) * 6 / mass)
            vl, wl = R[b].T @ v[b], R[b].T @ w[b]
            fl, tl = _drag(s, vl, wl, RHO, MU)
            power += fl @ vl + tl @ wl
        assert power < 0
        np.testing.assert_allclose(f @ qvel, power, rtol=1e-7)


def test_passive_switch_turns_the_medium_off():
    half = (0.03, 0.05, 0.08)
    qpos = np.r_[np.zeros(9), 0.3, 0.2, 1.0, 1.0, 0.0, 0.0, 0.0]
    qvel = np.r_[np.zeros(9), 1.0, -0.5, 0.2, 3.0, 1.0, -2.0]
    sc = _medium(_scene([_box(half)], qpos[9:]))
    sc.options.disableflags |= S.DISABLE_PASSIVE
    m, om, od = _oracle(sc)
    od['qvel'][:] = qvel
    od.forward(None, native.FLAG_NO_CONTROL)
    assert np.abs(od['qfrc_passive'][0]).max() == 0.0
