"""Pins of the oracle's contact-frame convention, with no code shared with the oracle.

The frame orients the friction pyramid and cone of every contact, so a slip in it changes the
physics of every config with friction.  The oracle restates the reference's contact_frame
(gpu/cuda/collision/mjwarp_contact.cuh:42-48): row 0 is the unit normal, row 1 the unit tangent
obtained from the world y axis (the world z axis when |n_y| >= 0.5) with its normal part removed,
row 2 their cross product; plane-capsule contacts take the capsule axis projected on the plane
as row 1 instead (gpu/cuda/collision/mjwarp_plane.cu:22-31).

* literal frames for normals along +-x, +-y, +-z and on both sides of |n_y| = 0.5, non-unit
  normals included;
* every frame a full oracle step publishes (family scene: plane, sphere, capsule, box and hull
  contacts; C3 and C1 scenes) is orthonormal and right-handed, row 0 along the contact's normal as
  the distance and positions define it;
* plane-capsule frames: row 1 is the capsule's published axis projected on the plane (sign kept).
"""
import numpy as np
import pytest

from oracle import oracle as O
from helpers import make_oracle

S2 = np.sqrt(2.0)


@pytest.mark.parametrize('normal,tangent,third', [
    ((1, 0, 0), (0, 1, 0), (0, 0, 1)),
    ((-1, 0, 0), (0, 1, 0), (0, 0, -1)),
    ((0, 1, 0), (0, 0, 1), (1, 0, 0)),
    ((0, -1, 0), (0, 0, 1), (-1, 0, 0)),
    ((0, 0, 1), (0, 1, 0), (-1, 0, 0)),
    ((0, 0, -1), (0, 1, 0), (1, 0, 0)),
    ((0, 0, 3.5), (0, 1, 0), (-1, 0, 0)),                          # not unit: normalised first
    ((1 / S2, 1 / S2, 0), (0, 0, 1), (1 / S2, -1 / S2, 0)),       # |n_y| > 0.5: from z
    ((0.6, 0.0, 0.8), (0, 1, 0), (-0.8, 0.0, 0.6)),
])
def test_literal_frames(normal, tangent, third):
    f = O.contact_frame(normal)
    n = np.asarray(normal, float) / np.linalg.norm(normal)
    np.testing.assert_allclose(f[0], n, atol=1e-15)
    np.testing.assert_allclose(f[1], tangent, atol=1e-15)
    np.testing.assert_allclose(f[2], third, atol=1e-15)


@pytest.mark.parametrize('ny', [0.49, 0.51, -0.49, -0.51])
def test_frames_either_side_of_the_switch(ny):
    """|n_y| just below 0.5 takes the tangent from y, just above from z."""
    n = np.array([np.sqrt(1 - ny * ny) * 0.6, ny, np.sqrt(1 - ny * ny) * 0.8])
    f = O.contact_frame(n)
    e = np.array([0.0, 1.0, 0.0]) if abs(ny) < 0.5 else np.array([0.0, 0.0, 1.0])
    other = np.array([0.0, 0.0, 1.0]) if abs(ny) < 0.5 else np.array([0.0, 1.0, 0.0])
    # the tangent lies in the plane of n and the chosen axis, on the axis' side, and is unit
    assert abs(np.dot(np.cross(n, e), f[1])) < 1e-15
    assert np.dot(f[1], e) > 0 and abs(np.linalg.norm(f[1]) - 1) < 1e-15
    assert abs(np.dot(f[1], n)) < 1e-15
    # with the other axis it would not lie in that plane
    assert abs(np.dot(np.cross(n, other), f[1])) > 0.1


def _published(scene, nworld, settle_steps=2):
    """Contacts of the last substep after a few oracle control steps from the scene's start."""
    from libero_hip.model import Model
    from libero_hip import scene as S
    m = Model(scene)
    om, od = make_oracle(m, nworld)
    od['qpos'][:] = scene.init_qpos
    od.forward(None, 8 | 2)
    acts = S.make_actions(nworld, settle_steps, seed=1)
    for a in acts:
        od['osc_action'][:] = a
        od.control_step(25, 1)
    return m, od


def _frames_are_orthonormal_right_handed(m, od, need_types=()):
    from libero_hip import scene as S
    gtype = m.arrays['geom_type']
    seen = set()
    count = 0
    for w in range(od.nworld):
        for i in range(int(od['ncon'][w, 0])):
            f = od['contact_frame'][w, 9 * i:9 * i + 9].reshape(3, 3)
            np.testing.assert_allclose(f @ f.T, np.eye(3), atol=1e-12)
            assert abs(np.linalg.det(f) - 1.0) < 1e-12
            g1, g2 = od['contact_geom'][w, 2 * i:2 * i + 2]
            seen.add((int(gtype[g1]), int(gtype[g2])))
            if gtype[g1] == S.PLANE:         # the plane's normal: its z axis, from geom 1 to geom 2
                np.testing.assert_allclose(f[0], od['geom_xmat'][w, 9 * g1:9 * g1 + 9].reshape(3, 3)[:, 2],
                                           atol=1e-12)
            count += 1
    for t in need_types:
        assert t in seen, (t, seen)
    return count, seen


def test_published_frames_family_scene():
    from libero_hip import scene as S
    from test_gpu_family_parity import family_scene
    nworld = 4
    m, od = _published(family_scene(nworld, seed=0), nworld)
    count, seen = _frames_are_orthonormal_right_handed(
        m, od, need_types=[(S.PLANE, S.CAPSULE), (S.PLANE, S.BOX), (S.PLANE, S.SPHERE), (S.SPHERE, S.BOX),
                           (S.CAPSULE, S.BOX), (S.BOX, S.BOX)])
    assert count > 20
    # plane-capsule: the second row is the capsule axis projected on the plane, normalised
    gtype = m.arrays['geom_type']
    checked = 0
    for w in range(nworld):
        for i in range(int(od['ncon'][w, 0])):
            g1, g2 = od['contact_geom'][w, 2 * i:2 * i + 2]
            if gtype[g1] != S.PLANE or gtype[g2] != S.CAPSULE:
                continue
            f = od['contact_frame'][w, 9 * i:9 * i + 9].reshape(3, 3)
            n = od['geom_xmat'][w, 9 * g1:9 * g1 + 9].reshape(3, 3)[:, 2]
            ax = od['geom_xmat'][w, 9 * g2:9 * g2 + 9].reshape(3, 3)[:, 2]
            t = ax - n * np.dot(n, ax)
            np.testing.assert_allclose(f[1], t / np.linalg.norm(t), atol=1e-12)
            np.testing.assert_allclose(f[2], np.cross(n, t / np.linalg.norm(t)), atol=1e-12)
            checked += 1
    assert checked >= nworld


@pytest.mark.parametrize('config', ['c3', 'c1'])
def test_published_frames_benchmark_scenes(config):
    """C3 (pyramidal: boxes, capsules, hulls on the table) and C1 (elliptic): every frame
    orthonormal and right-handed, and for non-plane contacts row 1 is the tangent of the y/z rule
    (in the plane of the normal and the chosen axis, on its side)."""
    from libero_hip import scene as S
    nworld = 4
    m, od = _published(S.make_scene(config, nworld, seed=0), nworld)
    count, _ = _frames_are_orthonormal_right_handed(m, od)
    assert count > 8
    for w in range(nworld):
        for i in range(int(od['ncon'][w, 0])):
            f = od['contact_frame'][w, 9 * i:9 * i + 9].reshape(3, 3)
            n = f[0]
            e = np.array([0.0, 1.0, 0.0]) if -0.5 < n[1] < 0.5 else np.array([0.0, 0.0, 1.0])
            assert abs(np.dot(np.cross(n, e), f[1])) < 1e-12 and np.dot(f[1], e) > 0
