"""The reference's GJK regression case: a real zero-margin box/box overlap from LIBERO-Spatial task 5
(substep 235, geoms 7 and 184) whose tuned support direction the reference once tested against the
preceding direction and so declared separated.  tests/golden/gjk_tuned_direction.json is the
reference's fixture (its tests/data/gjk_tuned_direction.json), kept as data.

The reference asserts that the pair overlaps by more than the tolerance and that the previously
claimed direction is not a separating plane (tests/test_mjwarp_convex_gjk.py:45-52).  Here:

* an independent 15-axis separating-axis test of the two boxes (face normals of both, the nine
  edge cross products) confirms both assertions and gives the penetration depth;
* the oracle's convex box-box route (GJK, EPA and the box manifold, the route a zero-margin box pair
  takes in this build) reports the contact at that depth, along the SAT axis; so does the
  primitive SAT route;
* on the GPU (marked gpu), the HIP kernel's narrowphase on the same pose, placed away from the arm
  as a static box and a free box, reports it too, within FP32 rounding of the SAT depth, and
  matches the oracle's contacts.
"""
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / 'golden'


def fixture():
    f = json.loads((GOLDEN / 'gjk_tuned_direction.json').read_text())
    a, b = np.asarray(f['position1']), np.asarray(f['position2'])
    ra, rb = (np.asarray(r) for r in f['rotations'])
    sa, sb = (np.asarray(s) for s in f['sizes'])
    return f, a, b, ra, rb, sa, sb


def sat(a, b, ra, rb, sa, sb):
    """Largest separation over the 15 candidate axes of two boxes (negative: penetration depth)
    and its unit axis, oriented from box a to box b."""
    axes = [ra[:, i] for i in range(3)] + [rb[:, i] for i in range(3)]
    axes += [np.cross(ra[:, i], rb[:, j]) for i in range(3) for j in range(3)]
    best, axis = -np.inf, None
    for ax in axes:
        n = np.linalg.norm(ax)
        if n < 1e-9:
            continue
        ax = ax / n
        gap = abs(ax @ (b - a)) - np.abs(ra.T @ ax) @ sa - np.abs(rb.T @ ax) @ sb
        if gap > best:
            best, axis = gap, ax * np.sign(ax @ (b - a))
    return best, axis


def test_fixture_is_an_overlap_and_the_old_direction_does_not_separate():
    f, a, b, ra, rb, sa, sb = fixture()
    depth, axis = sat(a, b, ra, rb, sa, sb)
    assert depth < -f['tolerance']
    d = np.asarray(f['previous_invalid_direction'])
    gap = d @ (a - b) - sum((np.abs(r.T @ d) @ s) for r, s in zip((ra, rb), (sa, sb)))
    assert f['previous_claimed_lower'] > 0 and gap < -f['tolerance']
    # the rotations are proper rotations (the fixture's FP32 matrices, to their rounding)
    for r in (ra, rb):
        assert np.abs(r @ r.T - np.eye(3)).max() < 1e-6 and abs(np.linalg.det(r) - 1) < 1e-6


@pytest.mark.parametrize('route,epa', [('convex', 16), ('convex', 35), ('primitive', None)])
def test_oracle_reports_the_penetration(route, epa):
    from oracle import oracle as O
    from libero_hip import scene as S
    f, a, b, ra, rb, sa, sb = fixture()
    depth, axis = sat(a, b, ra, rb, sa, sb)
    pos, normal, dist = O.collide(dict(type=S.BOX, pos=a, mat=ra, size=sa), dict(type=S.BOX, pos=b, mat=rb, size=sb),
                                  boxbox=route, iterations=f['iterations'], epa_iterations=epa)
    assert len(dist) >= 1 and (dist < 0).all()
    k = int(np.argmin(dist))
    assert abs(dist[k] - depth) < 1e-9
    np.testing.assert_allclose(normal[k], axis, atol=1e-9)
    # every contact point lies between the two boxes' surfaces along the normal: inside or on box a
    # expanded by the depth, and inside or on box b likewise
    for p in pos:
        for c, r, s in ((a, ra, sa), (b, rb, sb)):
            assert (np.abs(r.T @ (p - c)) <= s + abs(depth) + 1e-9).all()


def regression_scene(nworld, offset=(0.0, 3.0, 0.5)):
    """The fixture's pair away from the arm: box 1 a static geom of the world body, box 2 a free
    box at the fixture's relative pose (same rotations and sizes, translated by `offset`)."""
    from scipy.spatial.transform import Rotation
    from libero_hip import scene as S
    f, a, b, ra, rb, sa, sb = fixture()
    arm, actuators, osc, q_ready = S._arm()
    world = S._world(table=False)
    qa = Rotation.from_matrix(ra).as_quat()
    world.geoms.append(S.Geom(S.BOX, size=tuple(sa), pos=tuple(a + offset), quat=(qa[3], *qa[:3]), contype=0,
                              conaffinity=1))
    mass = 1000.0 * 8 * np.prod(sb)
    box = S.Body('fixture_box', 0, mass=mass, inertia=S.box_inertia(mass, tuple(sb)))
    box.geoms.append(S.Geom(S.BOX, size=tuple(sb)))
    box.joints.append(S.Joint(S.FREE))
    opts = S.Options()
    opts.cone, opts.nconmax = S.PYRAMIDAL, 16
    qb = Rotation.from_matrix(rb).as_quat()
    qpos = np.tile(np.r_[q_ready, 0.02, 0.02, b + offset, qb[3], qb[:3]], (nworld, 1))
    return S.Scene(name='gjk_regression', bodies=[world] + arm + [box], actuators=actuators, options=opts,
                   nworld=nworld, substeps=25, osc=osc, init_qpos=qpos, init_qvel=np.zeros((nworld, 15)), seed=0)


def scene_sat(m, geom_xpos, geom_xmat):
    """SAT of the scene's two fixture boxes at their published poses (the world's second geom and
    the last geom)."""
    g1, g2 = 1, m.ngeom - 1
    size = m.arrays['geom_size'].reshape(-1, 3)
    x = np.asarray(geom_xpos, float).reshape(-1, 3)
    r = np.asarray(geom_xmat, float).reshape(-1, 3, 3)
    return sat(x[g1], x[g2], r[g1], r[g2], size[g1], size[g2])


def test_regression_scene_on_the_oracle():
    """The full oracle forward pass on the scene: the pair's contacts at the SAT depth (the
    zero-margin box pair takes the convex route, EPA at 16 iterations)."""
    from helpers import make_oracle
    from libero_hip.model import Model
    m = Model(regression_scene(2))
    assert m.boxbox_primitive == 0
    om, od = make_oracle(m, 2)
    od['qpos'][:] = m.scene.init_qpos
    od.forward(None, 8 | 2)
    depth, axis = scene_sat(m, od['geom_xpos'][0], od['geom_xmat'][0])
    assert abs(depth - sat(*fixture()[1:])[0]) < 1e-8       # the pose went through a quaternion
    n = int(od['ncon'][0, 0])
    assert n >= 1
    dist = od['contact_dist'][0, :n]
    assert abs(dist.min() - depth) < 1e-9
    np.testing.assert_allclose(od['contact_frame'][0, 9 * int(np.argmin(dist)):][:3], axis, atol=1e-9)


@pytest.mark.gpu
def test_regression_scene_on_the_gpu(gpu_available):
    """The HIP kernel's forward pass on the fixture's pose (FP32 state): the contact is found, its
    depth within 2e-7 of the SAT depth of the oracle's geom poses from the same FP32-rounded state
    (the kernel's FP32 frames and narrowphase), its normal along the SAT axis within 1e-5, and the
    contact set equals the oracle's."""
    import torch
    from helpers import make_oracle
    from libero_hip import native
    from libero_hip.model import Model
    nworld = 4
    m = Model(regression_scene(nworld))
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld)
    q32 = m.scene.init_qpos.astype(np.float32)
    dd['qpos'].copy_(torch.from_numpy(q32))
    dd['body_active'].fill_(1)
    om, od = make_oracle(m, nworld)
    od['qpos'][:] = q32.astype(np.float64)
    dd.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    od.forward(None, 8 | 2)
    torch.cuda.synchronize()
    depth, axis = scene_sat(m, od['geom_xpos'][0], od['geom_xmat'][0])
    ncon = dd['ncon'].cpu().numpy()[:, 0]
    dist = dd['contact_dist'].double().cpu().numpy()
    frame = dd['contact_frame'].double().cpu().numpy()
    pos = dd['contact_pos'].double().cpu().numpy()
    for w in range(nworld):
        n = int(ncon[w])
        print('world', w, 'contacts', n, 'depth', dist[w, :n].min(), 'sat', depth, flush=True)
        assert n >= 1 and n == int(od['ncon'][w, 0])
        k = int(np.argmin(dist[w, :n]))
        assert abs(dist[w, k] - depth) < 2e-7
        np.testing.assert_allclose(frame[w, 9 * k:9 * k + 3], axis, atol=1e-5)
        np.testing.assert_allclose(dist[w, :n], od['contact_dist'][w, :n], rtol=0, atol=2e-7)
        np.testing.assert_allclose(pos[w, :3 * n], od['contact_pos'][w, :3 * n], rtol=0, atol=2e-5)
