"""Pins of the oracle's MPR convex narrowphase (MuJoCo 2.3.7 collision semantics, libccd's
ccdMPRPenetration) by geometry it does not compute:

* aligned cube hulls overlapping along one axis: the depth is the overlap, the normal that axis
  (from geom 1 to geom 2), the point halfway between the overlapping faces;
* a sphere resting into a hull's face: depth r - (centre height), the normal the face normal (the
  sphere's surface normal), the point on the segment between the surfaces;
* a sphere on a hull's corner (MPR's collinear branch): the vertex contact's closed form;
* a capsule lying in a hull's top face: depth and the capsule's radial normal;
* random hull pairs: moving geom 2 along the reported normal by the depth plus a margin separates
  the pair and by the depth minus it does not (GJK/EPA of the oracle's other route decides), and
  MPR's depth is never below the minimum penetration depth EPA finds.
"""
import numpy as np
import pytest

from oracle import oracle as O

SPHERE, CAPSULE, BOX, MESH = 2, 3, 6, 7


def _cube(half, pos, mat=np.eye(3)):
    v = np.array([[x, y, z] for x in (-1, 1) for y in (-1, 1) for z in (-1, 1)], float) * half
    return dict(type=MESH, pos=np.asarray(pos, float), mat=mat, vert=v)


ROUTES = ['mpr', 'mpr64']   # zero tests of the reference's FP32 route (the kernel's), of MuJoCo's double build


def _mpr(g1, g2, margin=0.0, route='mpr'):
    return O.collide(g1, g2, margin, convex=route, tolerance=1e-6, iterations=50)


@pytest.mark.parametrize('route', ROUTES)
@pytest.mark.parametrize('overlap', [0.002, 0.01, 0.03])
def test_aligned_cubes(overlap, route):
    h = 0.05
    a = _cube(h, (0.0, 0.0, 0.0))
    b = _cube(h, (2 * h - overlap, 0.01, -0.005))
    pos, nrm, dist = _mpr(a, b, route=route)
    assert len(dist) == 1
    np.testing.assert_allclose(dist[0], -overlap, atol=1e-9)
    np.testing.assert_allclose(nrm[0], [1.0, 0.0, 0.0], atol=1e-9)
    np.testing.assert_allclose(pos[0][0], h - overlap / 2, atol=1e-9)   # halfway between the faces
    # separated cubes: no contact; within the margin: a contact at the gap distance
    far = _cube(h, (2 * h + 0.004, 0.0, 0.0))
    assert len(_mpr(a, far, route=route)[2]) == 0
    pos, nrm, dist = _mpr(a, far, margin=0.01, route=route)
    np.testing.assert_allclose(dist, [0.004], atol=1e-9)


@pytest.mark.parametrize('route', ROUTES)
def test_sphere_into_hull_face(route):
    h, r = 0.05, 0.02
    cube = _cube(h, (0.0, 0.0, 0.0))
    for height in (0.015, 0.019):
        ball = dict(type=SPHERE, pos=(0.01, -0.02, h + height), size=(r, 0, 0))
        pos, nrm, dist = _mpr(ball, cube, route=route)        # pair order as the model sorts it (sphere first)
        assert len(dist) == 1
        np.testing.assert_allclose(dist[0], height - r, atol=1e-7)
        # from the sphere to the hull: the sphere's surface normal at the contact point, which MPR
        # locates on a curved side only to sqrt(2 tolerance / r) ~ 1e-2 rad of the portal spread
        np.testing.assert_allclose(nrm[0], [0.0, 0.0, -1.0], atol=2e-3)
        assert abs(pos[0][0] - 0.01) < r * 2e-2 and abs(pos[0][1] + 0.02) < r * 2e-2
        assert h + height - r - 1e-7 <= pos[0][2] <= h + 1e-7     # between the two surfaces


@pytest.mark.parametrize('route', ROUTES)
@pytest.mark.parametrize('offset', [0.0, 0.4])
def test_sphere_on_hull_corner(route, offset):
    """A sphere pressed onto a cube's corner from near the diagonal: the vertex contact's depth
    r - |c - corner| and normal (c - corner) / |c - corner|.  On the diagonal both routes take MPR's
    collinear branch (the centre ray passes through the support point); 0.4 degrees off it the FP32
    route's absolute zero test on the squared cross product still does, MuJoCo's double build refines
    a portal, and both stay within the closed form's first-order change."""
    h, r, pen = 0.05, 0.02, 0.003
    cube = _cube(h, (0.0, 0.0, 0.0))
    diag = np.ones(3) / np.sqrt(3.0)
    a = np.radians(offset)
    u = diag * np.cos(a) + np.array([1.0, -1.0, 0.0]) / np.sqrt(2.0) * np.sin(a)
    corner = np.full(3, h)
    centre = corner + u * (r - pen)
    pos, nrm, dist = _mpr(dict(type=SPHERE, pos=centre, size=(r, 0, 0)), cube, route=route)
    assert len(dist) == 1
    tol = 1e-9 if offset == 0.0 else 2e-4
    np.testing.assert_allclose(dist[0], -pen, atol=tol)
    np.testing.assert_allclose(nrm[0], -u, atol=1e-9 if offset == 0.0 else 1e-2)
    if offset == 0.0:   # the point halfway between the corner and the sphere's deepest point
        np.testing.assert_allclose(pos[0], corner - u * pen / 2, atol=1e-9)


@pytest.mark.parametrize('route', ROUTES)
def test_capsule_lying_in_hull_top(route):
    h, r, half = 0.05, 0.015, 0.03
    cube = _cube(h, (0.0, 0.0, 0.0))
    rx = np.array([[1, 0, 0], [0, 0, -1], [0, 1, 0]], float)        # capsule axis along world y
    cap = dict(type=CAPSULE, pos=(0.0, 0.0, h + r - 0.003), mat=rx, size=(r, half, 0))
    pos, nrm, dist = _mpr(cap, cube, route=route)
    assert len(dist) == 1
    np.testing.assert_allclose(dist[0], -0.003, atol=1e-7)
    # the capsule's radial normal at the contact point (located on the round side to the portal spread)
    np.testing.assert_allclose(nrm[0], [0.0, 0.0, -1.0], atol=2e-3)


def _hull(rng, n=20, scale=0.04):
    d = rng.normal(size=(n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    return d * scale * rng.uniform(0.6, 1.0, size=(n, 1))


def _rot(rng):
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


@pytest.mark.parametrize('route', ROUTES)
def test_random_hull_pairs_against_gjk_epa(route):
    rng = np.random.default_rng(17)
    checked = 0
    for trial in range(60):
        a = dict(type=MESH, pos=np.zeros(3), mat=_rot(rng), vert=_hull(rng))
        b = dict(type=MESH, pos=rng.normal(size=3) * 0.02, mat=_rot(rng), vert=_hull(rng))
        pos, nrm, dist = _mpr(a, b, route=route)
        gpos, gnrm, gdist = O.collide(a, b, boxbox='convex')
        if len(dist) == 0:
            # MPR found no penetration: GJK agrees that the hulls are apart (or barely touching)
            assert len(gdist) == 0 or gdist.min() > -1e-6
            continue
        depth, n = -dist[0], nrm[0]
        assert abs(np.linalg.norm(n) - 1) < 1e-9
        assert len(gdist) and depth >= -gdist.min() - 1e-6          # never below the minimum depth
        moved = dict(b, pos=b['pos'] + (depth + 1e-4) * n)
        assert len(O.collide(a, moved, boxbox='convex')[2]) == 0      # separated
        if depth > 2e-4:
            moved = dict(b, pos=b['pos'] + (depth - 1e-4) * n)
            assert len(O.collide(a, moved, boxbox='convex')[2]) > 0   # still penetrating
        checked += 1
    assert checked >= 20


def _margin_scene(gap_height, mpr):
    """A static box (margin 0.004, gap 0.001) with a cube hull (MPR under Options.mpr) and a free
    box (the primitive box-box routine) resting above its top face at `gap_height`, both with margin
    0.01 and gap 0.002, away from the arm."""
    from libero_hip import scene as S
    arm, actuators, osc, q_ready = S._arm()
    world = S._world(table=False)
    top = np.array([0.0, 3.0, 0.5])
    world.geoms.append(S.Geom(S.BOX, size=(0.2, 0.2, 0.02), pos=tuple(top - [0, 0, 0.02]), contype=0, conaffinity=1,
                              margin=0.004, gap=0.001))
    h = 0.02
    cube = np.array([[x, y, z] for x in (-1, 1) for y in (-1, 1) for z in (-1, 1)], float) * h
    mass = 1000.0 * 8 * h ** 3
    hull = S.Body('hull', 0, mass=mass, inertia=S.box_inertia(mass, (h, h, h)))
    hull.geoms.append(S.Geom(S.MESH, vertices=cube, margin=0.01, gap=0.002))
    hull.joints.append(S.Joint(S.FREE))
    box = S.Body('box', 0, mass=mass, inertia=S.box_inertia(mass, (h, h, h)))
    box.geoms.append(S.Geom(S.BOX, size=(h, h, h), margin=0.01, gap=0.002))
    box.joints.append(S.Joint(S.FREE))
    opts = S.Options()
    opts.mpr, opts.cone, opts.nconmax = mpr, S.PYRAMIDAL, 16
    z = top[2] + h + gap_height
    qpos = np.r_[q_ready, 0.02, 0.02, -0.1, 3.0, z, 1, 0, 0, 0, 0.1, 3.0, z, 1, 0, 0, 0][None]
    return S.Scene(name='margins', bodies=[world] + arm + [hull, box], actuators=actuators, options=opts, nworld=1,
                   substeps=25, osc=osc, init_qpos=qpos, init_qvel=np.zeros((1, 21)), seed=0)


@pytest.mark.parametrize('mpr', [True, False])
def test_margin_and_gap_combination(mpr):
    """MuJoCo 2.3.7 (Options.mpr; mj_collideGeoms, the reference's native route
    collision/collision_dispatch.cuh:115-116): a pair's margin is the larger geom margin (0.01), its
    gap the larger gap (0.002); contacts are detected below the margin and their rows use margin - gap
    (0.008).  The MJWarp route (mjwarp_contact.cuh:71-72): margins and gaps add (0.014, 0.003),
    detection below their sum (0.017), rows at 0.011.  A pair 0.012 apart, between the larger margin
    and the summed one, has contacts only on the MJWarp route; one 0.006 apart has them on both, at
    that distance (within MPR's tolerance)."""
    from helpers import make_oracle
    from libero_hip.model import Model
    from libero_hip import scene as S
    for height, expect in ((0.012, not mpr), (0.006, True), (0.0125, not mpr), (0.016, not mpr), (0.018, False)):
        m = Model(_margin_scene(height, mpr))
        assert m.convex_mpr == int(mpr) and m.boxbox_primitive == 1
        om, od = make_oracle(m, 1)
        od['qpos'][:] = m.scene.init_qpos
        od.forward(None, 8 | 2)
        n = int(od['ncon'][0, 0])
        gtype = m.arrays['geom_type']
        pairs = {int(gtype[g]) for g in od['contact_geom'][0, 1:2 * n:2]}
        assert (n > 0) == expect, (height, n)
        if expect:
            assert pairs == {S.MESH, S.BOX}, pairs             # both the MPR pair and the box-box pair
            # (MPR stops within its tolerance, 1e-6; the primitive box-box is exact)
            np.testing.assert_allclose(od['contact_dist'][0, :n], height, atol=1e-6)
            np.testing.assert_allclose(od['contact_includemargin'][0, :n], 0.008 if mpr else 0.011, atol=1e-15)
