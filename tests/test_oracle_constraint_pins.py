"""Pins of the oracle's constraint-row force law, contact materials, actuators and broadphase.

None of these checks shares code with the oracle.  The oracle restates the reference's row build
(gpu/cuda/dynamics/mjwarp_constraint_build.cu:22-48 impedance and publish_row, :161-199 contact
rows), its material mixing (gpu/cuda/collision/mjwarp_contact.cuh:56-101), actuator forces
(gpu/cuda/fp32/fused_control_drive.cu) and broadphase (gpu/cuda/collision/mjwarp_broadphase.cu).
They are pinned here by what MuJoCo documents those numbers to mean:

* solref = (timeconst, dampratio): with a flat impedance d = dmin = dmax, a violated constraint on
  one dof moves as the mass-spring-damper  a = (1 - d) a0 - (2 / timeconst) v - r / (timeconst
  dampratio)^2  (natural frequency 1 / (timeconst dampratio), damping ratio dampratio; the
  unconstrained acceleration a0 passes with weight 1 - d).  The oracle's trajectory of a limited
  slide joint and of a frictionless sphere on the ground plane must follow the semi-implicit Euler
  recursion of that ODE step by step.  A missing impedance factor, a wrong damping or stiffness
  formula, a wrong regularizer R = (1 - d) / d * A or a wrong contact depth fails it.
* solref = (-stiffness, -damping) (direct format): at full impedance (|r| >= width) the constraint
  is the spring-damper a = -stiffness r - damping v; below it the stiffness is scaled by
  (d(r) / dmax)^2, which recovers the impedance curve d(r) from the accelerations at rest.
* solimp = (dmin, dmax, width, mid, power): d(0) = dmin, d(|r| >= width) = dmax, the curve passes
  through dmin + mid (dmax - dmin) at |r| = mid width, grows as x^power below mid and approaches
  dmax as (1 - x)^power above it, and is linear for power 1 (MuJoCo's documented sigmoid).
  Swapped dmin / dmax, a wrong branch or a wrong exponent fails these shape checks.
* Elliptic cones: impratio is the ratio of frictional to normal impedance (friction rows' D =
  impratio times the normal row's D for isotropic tangential friction), and friction rows carry
  damping only: aref = -b v_t with the normal row's b.
* Pyramidal cones: edge rows J_n +- mu J_t carry the position term of the normal row; each edge's
  regularizer uses the weight A (1 + mu^2) 2 mu^2 / impratio (the reference's line 176-182); at rest
  the four edges of a sphere share its weight equally.
* Materials: MuJoCo's documented mixing rule (higher priority wins friction and condim, solmix
  weights solref / solimp otherwise with the 0 / 0.5 special cases, element-wise minimum for direct
  solref, friction and condim by maximum).
* Actuators: motor force = gain ctrl (ctrl clamped to ctrlrange), position servo force =
  kp (ctrl - q) - kv qdot clamped to forcerange, generalized force = gear * force.
* Broadphase: on random states (overlapping, touching and separated objects) the contacts of a
  full step equal those of the narrowphase run on every pair of the static pair table.
"""
import math

import numpy as np
import pytest

from libero_hip import native, scene as S
from libero_hip.model import Model
from helpers import make_oracle
from oracle import oracle as O

G = 9.81
H = 0.002


def _scene(objects, obj_qpos, *, nworld=1, cone=S.PYRAMIDAL, gravity=(0.0, 0.0, -G), impratio=20.0,
           nconmax=8, world_geoms=None):
    """The arm (required by the controller, parked) on a bare ground plane, plus `objects`."""
    arm, actuators, osc, q_ready = S._arm()
    world = S._world(table=False)
    if world_geoms is not None:
        world.geoms = world_geoms
    bodies = [world] + arm + list(objects)
    opts = S.Options()
    opts.cone, opts.gravity, opts.impratio, opts.nconmax = cone, gravity, impratio, nconmax
    nq_obj = sum(7 if j.type == S.FREE else 1 for b in objects for j in b.joints)
    qpos = np.zeros((nworld, 9 + nq_obj))
    qpos[:, :7] = q_ready
    qpos[:, 7:9] = 0.02                     # fingers inside their limits
    qpos[:, 9:] = obj_qpos
    return S.Scene(name='pin', bodies=bodies, actuators=actuators, options=opts, nworld=nworld, substeps=1,
                   osc=osc, init_qpos=qpos, init_qvel=np.zeros((nworld, 9 + sum(
                       6 if j.type == S.FREE else 1 for b in objects for j in b.joints))))


def _oracle(sc):
    m = Model(sc)
    om, od = make_oracle(m, sc.nworld)
    od['qpos'][:] = sc.init_qpos
    od['qvel'][:] = sc.init_qvel
    return m, om, od


def _slider(mass, solref, solimp, lo=0.0):
    """A body on a vertical slide joint limited below at `lo` (no geom): one dof, M = mass."""
    b = S.Body('slider', 0, pos=(0.0, 1.5, 0.5), mass=mass, inertia=(0.01, 0.01, 0.01))
    b.joints.append(S.Joint(S.SLIDE, axis=(0.0, 0.0, 1.0), limited=True, range=(lo, 1.0),
                            solref=solref, solimp=solimp))
    return b


def _sphere(mass, radius, *, condim=1, friction=(1.0, 0.005, 0.0001), solref=S.SOLREF_DEFAULT,
            solimp=S.SOLIMP_DEFAULT, priority=0, solmix=1.0):
    inertia = (0.4 * mass * radius ** 2,) * 3
    b = S.Body('ball', 0, mass=mass, inertia=inertia)
    b.geoms.append(S.Geom(S.SPHERE, size=(radius, 0.0, 0.0), condim=condim, friction=friction,
                          solref=solref, solimp=solimp, priority=priority, solmix=solmix))
    b.joints.append(S.Joint(S.FREE))
    return b


def _msd_trajectory(r0, v0, a0, d, timeconst, dampratio, steps):
    """Semi-implicit Euler of a = (1 - d) a0 - (2 / timeconst) v - r / (timeconst dampratio)^2."""
    r, v, out = r0, v0, []
    for _ in range(steps):
        a = (1.0 - d) * a0 - 2.0 / timeconst * v - r / (timeconst * dampratio) ** 2
        v = v + H * a
        r = r + H * v
        out.append(r)
    return np.array(out)


# ------------------------------------------------------------------ solref / solimp semantics
@pytest.mark.parametrize('timeconst,dampratio,d', [(0.1, 0.5, 0.9), (0.05, 1.0, 0.95), (0.2, 0.3, 0.5)])
def test_limit_row_is_the_documented_mass_spring_damper(timeconst, dampratio, d):
    mass = 2.0
    eq = -(1.0 - d) * G * (timeconst * dampratio) ** 2      # resting penetration of the ODE
    sc = _scene([_slider(mass, (timeconst, dampratio), (d, d, 0.001, 0.5, 2.0))], [2.0 * eq])
    m, om, od = _oracle(sc)
    steps = 150
    got = []
    for _ in range(steps):
        od.control_step(1, native.FLAG_NO_CONTROL)
        got.append(od['qpos'][0, 9])
    want = _msd_trajectory(2.0 * eq, 0.0, -G, d, timeconst, dampratio, steps)
    assert (want < 0).all()                                   # the limit stays violated
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-10 * abs(eq))
    assert abs(got[-1] - eq) < 0.2 * abs(eq) or dampratio < 0.5


def test_frictionless_contact_is_the_documented_mass_spring_damper():
    """The same law through the collision path: a sphere (condim 1) penetrating the ground plane;
    the contact's Jacobian is the sphere's vertical dof and its weight 1 / mass."""
    mass, radius, timeconst, dampratio, d = 0.7, 0.05, 0.08, 0.6, 0.9
    eq = -(1.0 - d) * G * (timeconst * dampratio) ** 2
    plane = S.Geom(S.PLANE, size=(0.0, 0.0, 1.0), contype=0, conaffinity=1, condim=1,
                   solref=(timeconst, dampratio), solimp=(d, d, 0.001, 0.5, 2.0))
    sc = _scene([_sphere(mass, radius, solref=(timeconst, dampratio), solimp=(d, d, 0.001, 0.5, 2.0))],
                [0.3, 0.2, radius + 2.0 * eq, 1.0, 0.0, 0.0, 0.0], cone=S.ELLIPTIC, world_geoms=[plane])
    m, om, od = _oracle(sc)
    steps = 150
    got = []
    for _ in range(steps):
        od.control_step(1, native.FLAG_NO_CONTROL)
        got.append(od['qpos'][0, 11] - radius)
        assert od['ncon'][0, 0] == 1 and od['contact_dim'][0, 0] == 1
    want = _msd_trajectory(2.0 * eq, 0.0, -G, d, timeconst, dampratio, steps)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-10 * abs(eq))


SOLIMP = (0.3, 0.95, 0.01, 0.4, 3.0)


def _impedance_from_rest(solimp, xs, stiffness=400.0, damping=30.0, velocity=0.0):
    """d(|r| = x width) recovered from the slider's acceleration with the direct-format solref
    (-stiffness, -damping), no gravity: a = -(d / dmax) damping v - (d / dmax)^2 stiffness r."""
    width, dmax = solimp[2], solimp[1]
    rs = -np.asarray(xs, float) * width
    sc = _scene([_slider(1.0, (-stiffness, -damping), solimp)], rs[:, None], nworld=len(rs),
                gravity=(0.0, 0.0, 0.0))
    m, om, od = _oracle(sc)
    od['qvel'][:, 9] = velocity
    od.forward(None, native.FLAG_NO_CONTROL)
    assert (od['nefc'][:, 0] == 1).all() and (od['efc_type'][:, 0] == 3).all()
    acc = od['qacc'][:, 9]
    return rs, acc, dmax * np.sqrt(acc / (-stiffness * rs)) if velocity == 0.0 else None


def test_direct_solref_is_a_spring_damper_at_full_impedance():
    stiffness, damping, v = 400.0, 30.0, 0.07
    rs, acc, _ = _impedance_from_rest(SOLIMP, [1.0, 1.5, 3.0], stiffness, damping, velocity=v)
    np.testing.assert_allclose(acc, -stiffness * rs - damping * v, rtol=1e-12)


def test_impedance_curve_shape():
    dmin, dmax, width, mid, power = SOLIMP
    xs = [1e-6, 0.1, 0.2, 0.3, mid, 0.6, 0.7, 0.9, 1.0, 2.0]
    _, _, d = _impedance_from_rest(SOLIMP, xs)
    d = dict(zip(xs, d))
    assert abs(d[1e-6] - dmin) < 1e-9                          # d(0) = dmin
    assert abs(d[1.0] - dmax) < 1e-12 and abs(d[2.0] - dmax) < 1e-12
    assert abs(d[mid] - (dmin + mid * (dmax - dmin))) < 1e-12   # through (mid, mid)
    vals = [d[x] for x in xs]
    assert all(b >= a for a, b in zip(vals, vals[1:]))         # monotone
    # power law on both sides of mid
    assert abs((d[0.2] - dmin) / (d[0.1] - dmin) - 2.0 ** power) < 1e-9
    assert abs((d[0.3] - dmin) / (d[0.1] - dmin) - 3.0 ** power) < 1e-9
    assert abs((dmax - d[0.9]) / (dmax - d[0.7]) - (0.1 / 0.3) ** power) < 1e-9
    assert abs((dmax - d[0.6]) / (dmax - d[0.7]) - (0.4 / 0.3) ** power) < 1e-9
    # power 1: a straight line from dmin to dmax
    lin = (dmin, dmax, width, mid, 1.0)
    _, _, dl = _impedance_from_rest(lin, [0.1, 0.25, 0.8])
    np.testing.assert_allclose(dl, dmin + np.array([0.1, 0.25, 0.8]) * (dmax - dmin), rtol=1e-12)
    # dmin = dmax: constant
    _, _, dc = _impedance_from_rest((0.7, 0.7, width, mid, power), [0.1, 0.5, 2.0])
    np.testing.assert_allclose(dc, 0.7, rtol=1e-12)


# ------------------------------------------------------------------ cone rows
def _penetrating_ball(cone, *, impratio, friction, vel=(0.0, 0.0, 0.0), depth=1e-3, nworld=1):
    """A sphere 1 mm into the ground plane, both geoms with `friction`."""
    radius, mass = 0.05, 0.7
    plane = S.Geom(S.PLANE, size=(0.0, 0.0, 1.0), contype=0, conaffinity=1, friction=friction)
    sc = _scene([_sphere(mass, radius, condim=3, friction=friction)],
                [0.3, 0.2, radius - depth, 1.0, 0.0, 0.0, 0.0], cone=cone, impratio=impratio, nworld=nworld,
                world_geoms=[plane])
    m, om, od = _oracle(sc)
    od['qvel'][:, 9:12] = vel
    od.forward(None, native.FLAG_NO_CONTROL)
    return m, od, mass


def _documented_kbd(solref, solimp, r):
    """MuJoCo's documented stiffness, damping and impedance for solref (timeconst, dampratio)."""
    dmin, dmax, width, mid, power = solimp
    timeconst = max(solref[0], 2 * H)
    k = 1.0 / (dmax * timeconst * solref[1]) ** 2
    b = 2.0 / (dmax * timeconst)
    x = min(abs(r) / width, 1.0)
    if x < mid:
        y = x ** power / mid ** (power - 1)
    else:
        y = 1 - (1 - x) ** power / (1 - mid) ** (power - 1)
    return k, b, dmin + y * (dmax - dmin)


@pytest.mark.parametrize('impratio', [1.0, 20.0, 7.5])
def test_elliptic_friction_rows(impratio):
    m, od, mass = _penetrating_ball(S.ELLIPTIC, impratio=impratio, friction=(0.8, 0.005, 0.0001),
                                    vel=(0.1, -0.04, 0.0))
    assert od['ncon'][0, 0] == 1 and od['nefc'][0, 0] == 3
    assert (od['efc_type'][0, :3] == 7).all()
    D, aref = od['efc_D'][0, :3], od['efc_aref'][0, :3]
    np.testing.assert_allclose(D[1:] / D[0], impratio, rtol=1e-12)
    r = od['contact_dist'][0, 0]
    k, b, d = _documented_kbd(S.SOLREF_DEFAULT, S.SOLIMP_DEFAULT, r)
    frame = od['contact_frame'][0, :9].reshape(3, 3)
    v = np.array([0.1, -0.04, 0.0])
    np.testing.assert_allclose(aref[0], -b * frame[0] @ v - k * d * r, rtol=1e-12)
    np.testing.assert_allclose(aref[1:], -b * frame[1:] @ v, rtol=1e-12, atol=1e-15)   # damping only
    np.testing.assert_allclose(D[0], d / ((1 - d) / mass), rtol=1e-12)            # weight 1 / mass
    assert od['efc_pos'][0, 1] == od['contact_includemargin'][0, 0]               # no position term


@pytest.mark.parametrize('mu,impratio', [(1.0, 1.0), (0.5, 20.0), (1.5, 4.0)])
def test_pyramidal_edge_rows(mu, impratio):
    vel = (0.1, -0.04, 0.02)
    m, od, mass = _penetrating_ball(S.PYRAMIDAL, impratio=impratio, friction=(mu, 0.005, 0.0001), vel=vel)
    assert od['nefc'][0, 0] == 4 and (od['efc_type'][0, :4] == 6).all()
    assert od['contact_friction'][0, 0] == mu
    D, aref = od['efc_D'][0, :4], od['efc_aref'][0, :4]
    r = od['contact_dist'][0, 0]
    k, b, d = _documented_kbd(S.SOLREF_DEFAULT, S.SOLIMP_DEFAULT, r)
    weight = (1.0 / mass) * (1 + mu * mu) * 2 * mu * mu / impratio
    np.testing.assert_allclose(D, d / ((1 - d) * weight), rtol=1e-12)
    frame = od['contact_frame'][0, :9].reshape(3, 3)
    v = np.array(vel)
    edges = [frame[0] + s * mu * frame[t] for t in (1, 2) for s in (1, -1)]
    np.testing.assert_allclose(aref, [-b * e @ v - k * d * r for e in edges], rtol=1e-11)


def test_pyramidal_edges_share_a_resting_weight():
    """A sphere settled on the plane: the four edge forces are equal and sum to its weight."""
    radius, mass = 0.05, 0.7
    sc = _scene([_sphere(mass, radius, condim=3)], [0.3, 0.2, radius - 1e-4, 1.0, 0.0, 0.0, 0.0])
    m, om, od = _oracle(sc)
    for _ in range(8):
        od.control_step(25, native.FLAG_NO_CONTROL)
    f = od['efc_force'][0, :4]
    assert od['nefc'][0, 0] == 4
    np.testing.assert_allclose(f.sum(), mass * G, rtol=1e-6)
    np.testing.assert_allclose(f, f.mean(), rtol=1e-6)


# ------------------------------------------------------------------ materials
def _mixed(plane_kw, ball_kw):
    """Contact material between the ground plane (geom 1) and a resting sphere (geom 2)."""
    radius = 0.05
    plane = S.Geom(S.PLANE, size=(0.0, 0.0, 1.0), contype=0, conaffinity=1, **plane_kw)
    sc = _scene([_sphere(0.7, radius, **ball_kw)], [0.3, 0.2, radius - 1e-3, 1.0, 0.0, 0.0, 0.0],
                world_geoms=[plane], cone=S.ELLIPTIC)
    m, om, od = _oracle(sc)
    od.forward(None, native.FLAG_NO_CONTROL)
    assert od['ncon'][0, 0] == 1
    return od


def _documented_mix(g1, g2):
    """MuJoCo's contact parameter mixing for geoms g1, g2 (dicts of priority, solmix, friction,
    condim, solref, solimp)."""
    if g1['priority'] != g2['priority']:
        win = g1 if g1['priority'] > g2['priority'] else g2
        mix = 1.0 if win is g1 else 0.0
        friction, condim = np.array(win['friction']), win['condim']
    else:
        friction = np.maximum(g1['friction'], g2['friction'])
        condim = max(g1['condim'], g2['condim'])
        s1, s2 = g1['solmix'], g2['solmix']
        if s1 < 1e-15 and s2 < 1e-15:
            mix = 0.5
        elif s1 < 1e-15:
            mix = 0.0
        elif s2 < 1e-15:
            mix = 1.0
        else:
            mix = s1 / (s1 + s2)
    r1, r2 = np.array(g1['solref']), np.array(g2['solref'])
    solref = mix * r1 + (1 - mix) * r2 if r1[0] > 0 and r2[0] > 0 else np.minimum(r1, r2)
    solimp = mix * np.array(g1['solimp']) + (1 - mix) * np.array(g2['solimp'])
    return friction, condim, solref, solimp


BASE = dict(priority=0, solmix=1.0, friction=(1.0, 0.005, 0.0001), condim=3, solref=(0.02, 1.0),
            solimp=(0.9, 0.95, 0.001, 0.5, 2.0))


@pytest.mark.parametrize('case', ['solmix', 'priority_ball', 'priority_plane', 'solmix_zero', 'both_zero',
                                  'direct_solref', 'condim_max'])
def test_material_mixing_follows_the_documented_rule(case):
    plane = dict(BASE)
    ball = dict(BASE, friction=(0.6, 0.01, 0.0003), solref=(0.04, 0.7), solimp=(0.8, 0.99, 0.002, 0.3, 3.0))
    if case == 'solmix':
        plane['solmix'], ball['solmix'] = 1.0, 3.0
    elif case == 'priority_ball':
        ball['priority'] = 2
    elif case == 'priority_plane':
        plane['priority'], ball['condim'] = 1, 1
    elif case == 'solmix_zero':
        ball['solmix'] = 0.0
    elif case == 'both_zero':
        plane['solmix'] = ball['solmix'] = 0.0
    elif case == 'direct_solref':
        ball['solref'] = (-2000.0, -40.0)
    elif case == 'condim_max':
        plane['condim'] = 1
    od = _mixed(plane, ball)
    friction, condim, solref, solimp = _documented_mix(plane, ball)
    assert od['contact_dim'][0, 0] == condim
    fr = od['contact_friction'][0, :5]
    np.testing.assert_allclose(fr, [friction[0], friction[0], friction[1], friction[2], friction[2]], rtol=1e-12)
    # the normal row's D and aref follow the mixed solref / solimp (qvel = 0: aref = -k d r)
    r = od['contact_dist'][0, 0]
    dmin, dmax, width, mid, power = solimp
    if solref[0] > 0:
        k, b, d = _documented_kbd(solref, solimp, r)
    else:
        _, _, d = _documented_kbd((0.02, 1.0), solimp, r)
        k = -solref[0] / dmax ** 2
    np.testing.assert_allclose(od['efc_aref'][0, 0], -k * d * r, rtol=1e-12)
    weight = 1.0 / 0.7
    if condim == 3:      # elliptic normal row: weight alone
        np.testing.assert_allclose(od['efc_D'][0, 0], d / ((1 - d) * weight), rtol=1e-12)


# ------------------------------------------------------------------ actuators
def test_actuator_forces_closed_form():
    """Motors: force = ctrl clamped to ctrlrange; finger position servos: kp (ctrl - q) - kv qdot
    clamped to forcerange; qfrc_actuator = gear * force on the joint's dof."""
    sc = S.make_scene('c1', 4, seed=0)
    m, om, od = _oracle(sc)
    rng = np.random.default_rng(5)
    od['qpos'][:, 7:9] = rng.uniform(0.0, 0.04, size=(4, 2))
    od['qvel'][:, :9] = rng.uniform(-1, 1, size=(4, 9))
    ctrl = np.zeros((4, 9))
    ctrl[:, :7] = rng.uniform(-150, 150, size=(4, 7))       # beyond some motors' ranges
    ctrl[:, 7:] = rng.uniform(-0.05, 0.09, size=(4, 2))     # beyond the servos' ctrlrange
    od['ctrl'][:] = ctrl
    od.forward(None, native.FLAG_NO_CONTROL)
    lo, hi = np.array([a.ctrlrange for a in sc.actuators]).T
    c = np.clip(ctrl, lo, hi)
    want = np.zeros((4, 9))
    for i, ac in enumerate(sc.actuators):
        q, qd = od['qpos'][:, ac.joint], od['qvel'][:, ac.joint]
        if ac.kind == 'motor':
            want[:, i] = c[:, i]
        else:
            f = ac.kp * c[:, i] - ac.kp * q - ac.kv * qd
            want[:, i] = np.clip(f, *ac.forcerange) if ac.forcelimited else f
    np.testing.assert_allclose(od['actuator_force'], want, rtol=1e-13, atol=1e-12)
    gear = np.array([a.gear for a in sc.actuators])
    np.testing.assert_allclose(od['qfrc_actuator'][:, :9], gear * want, rtol=1e-13, atol=1e-12)
    assert (np.abs(want[:, 7:]) == 20.0).any()              # some servo hit its force limit


# ------------------------------------------------------------------ broadphase
def _geom_dict(m, od, w, g):
    a = m.arrays
    t = int(a['geom_type'][g])
    d = dict(type=t, pos=od['geom_xpos'][w, 3 * g:3 * g + 3], mat=od['geom_xmat'][w, 9 * g:9 * g + 9].reshape(3, 3),
             size=a['geom_size'][g])
    if t == S.MESH:
        mid = int(a['geom_dataid'][g])
        adr, n = int(a['mesh_vertadr'][mid]), int(a['mesh_vertnum'][mid])
        d['vert'] = a['mesh_vert'].reshape(-1, 3)[adr:adr + n]
    return d


@pytest.mark.parametrize('config', ['c3', 'c1'])
def test_broadphase_drops_no_contact(config):
    sc = S.make_scene(config, 24, seed=11)
    m = Model(sc)
    om, od = make_oracle(m, 24)
    rng = np.random.default_rng(12)
    qpos = sc.init_qpos.copy()
    nobj = (m.nq - 9) // 7
    for w in range(24):
        for k in range(nobj):   # objects clustered above the table: overlapping, touching, apart
            qpos[w, 9 + 7 * k:12 + 7 * k] = (0.55 + rng.uniform(-0.12, 0.12), rng.uniform(-0.12, 0.12),
                                             0.8 + rng.uniform(-0.01, 0.12))
            q = rng.normal(size=4)
            qpos[w, 12 + 7 * k:16 + 7 * k] = q / np.linalg.norm(q)
    od['qpos'][:] = qpos
    od.forward(None, native.FLAG_NO_CONTROL)
    a = m.arrays
    total = 0
    for w in range(24):
        want = {}
        for g1, g2 in a['pair_geom']:
            margin = a['geom_margin'][g1] + a['geom_margin'][g2]
            gap = a['geom_gap'][g1] + a['geom_gap'][g2]
            p, n, d = O.collide(_geom_dict(m, od, w, g1), _geom_dict(m, od, w, g2), margin, gap=gap,
                                boxbox='primitive' if m.boxbox_primitive else 'convex',
                                epa_iterations=m.epa_iterations, iterations=sc.options.ccd_iterations)
            if len(d):
                want[(int(g1), int(g2))] = np.sort(d)
        nc = int(od['ncon'][w, 0])
        got = {}
        geoms = od['contact_geom'][w, :2 * nc].reshape(-1, 2)
        for i in range(nc):
            got.setdefault(tuple(int(x) for x in geoms[i]), []).append(od['contact_dist'][w, i])
        assert set(got) == set(want), (w, set(want) - set(got))
        for key in want:
            np.testing.assert_allclose(np.sort(got[key]), want[key], rtol=0, atol=1e-12)
        total += nc
    assert total > 24
