"""CPU checks that pin the oracle's narrowphase (no GPU).

Each primitive pair is checked against geometry it does not share code with: closed forms for
plane contacts, brute-force sampled signed distances for sphere/capsule/box pairs, an independent
15-axis separating-axis test for box-box existence and depth, and the reference's own box-box
regression fixtures (tests/golden/boxbox_*, copied as data from the reference's tests/fixtures/,
used by its tests/test_native_box_contacts.py:140-255).

Contact convention under test (MuJoCo): the normal points from geom 1 to geom 2, ``dist < 0`` is
penetration, ``pos`` is the midpoint, so the surface witness of geom 1 is ``pos - dist/2 n`` and
that of geom 2 is ``pos + dist/2 n``.

Box-box conventions differ between the reference's collision routes: its MuJoCo-native route
(the one the fixtures were captured on) reports half the penetration for face contacts
(tests/fixtures/boxbox_sat_face_tie.csv: -0.007675 for a 0.01535 overlap) and up to eight
raw points, while its product routes (primitive ``box_box``, gpu/cuda/collision/mjwarp_box.cu:115-176,
and the convex box manifold) report the full depth and at most four face points or one edge
point.  The assertions below are the route-independent ones: witnesses on the boxes, existence,
depth bounds, counts for face contacts.
"""
import csv
import json
from pathlib import Path

import numpy as np
import pytest

from libero_hip.model import quat2mat
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / 'golden'
PLANE, SPHERE, CAPSULE, BOX = 0, 2, 3, 6


def rot(rng):
    q = rng.normal(size=4)
    return quat2mat(q / np.linalg.norm(q))


def signed_point_box(p, c, R, h):
    """Signed distance of point p to the box (centre c, rotation R, half sizes h)."""
    local = R.T @ (np.asarray(p) - c)
    q = np.clip(local, -h, h)
    out = np.linalg.norm(local - q)
    return out if out > 0 else -np.min(h - np.abs(local))


def seg_points(c, R, half, n):
    t = np.linspace(-1, 1, n)
    return c[None, :] + t[:, None] * half * R[:, 2][None, :]


def boxes(size, pos, mat):
    return [dict(type=BOX, pos=pos[k], mat=np.asarray(mat[k]).reshape(3, 3), size=size[k]) for k in range(2)]


def box_witnesses_ok(p, n, d, size, pos, mat, tol):
    for k, sgn in ((0, -1), (1, 1)):
        w = p + sgn * 0.5 * d[:, None] * n
        local = (w - pos[k]) @ np.asarray(mat[k]).reshape(3, 3)
        if not np.all(np.abs(local) <= np.asarray(size[k]) + tol):
            return False
        if not np.all(np.min(np.abs(np.abs(local) - size[k]), axis=1) < tol):
            return False
    return True


def sat_depth(size, pos, mat):
    """Independent separating-axis test: min over 15 axes of the projected overlap."""
    A = [np.asarray(mat[k]).reshape(3, 3) for k in range(2)]
    axes = [A[0][:, i] for i in range(3)] + [A[1][:, i] for i in range(3)]
    for i in range(3):
        for j in range(3):
            c = np.cross(A[0][:, i], A[1][:, j])
            if np.linalg.norm(c) > 1e-6:
                axes.append(c / np.linalg.norm(c))
    d = np.asarray(pos[1]) - np.asarray(pos[0])
    best = np.inf
    for L in axes:
        r = sum(np.sum(np.asarray(size[k]) * np.abs(A[k].T @ L)) for k in range(2))
        best = min(best, r - abs(d @ L))
    return best          # > 0: overlap depth, < 0: separated


# ------------------------------------------------------------------------------ plane
def test_plane_sphere_closed_form():
    for z, r in ((0.3, 0.5), (0.05, 0.04), (-0.1, 0.2)):
        p, n, d = O.collide(dict(type=PLANE, pos=[0, 0, 0]), dict(type=SPHERE, pos=[0.2, -0.1, z], size=[r]))
        if z - r >= 0:
            assert len(d) == 0
            continue
        np.testing.assert_allclose(d, [z - r], atol=1e-15)
        np.testing.assert_allclose(n[0], [0, 0, 1], atol=1e-15)
        np.testing.assert_allclose(p[0], [0.2, -0.1, (z - r) / 2], atol=1e-15)


def test_plane_capsule_endpoints():
    rng = np.random.default_rng(1)
    for _ in range(20):
        R = rot(rng)
        c = np.array([0.1, 0.2, rng.uniform(-0.05, 0.2)])
        r, half = 0.04, 0.1
        ends = [c - half * R[:, 2], c + half * R[:, 2]]
        p, n, d = O.collide(dict(type=PLANE, pos=[0, 0, 0]), dict(type=CAPSULE, pos=c, mat=R, size=[r, half]))
        expect = sorted(e[2] - r for e in ends if e[2] - r < 0)
        np.testing.assert_allclose(sorted(d), expect, atol=1e-15)
        for k in range(len(d)):
            np.testing.assert_allclose(n[k], [0, 0, 1], atol=1e-15)


def test_plane_box_every_corner_below_threshold():
    # the reference emits each of the 8 corners under margin + gap, in corner order
    # (gpu/cuda/collision/mjwarp_plane.cu:32-39)
    rng = np.random.default_rng(2)
    h = np.array([0.05, 0.08, 0.03])
    for margin in (0.0, 0.01):
        for _ in range(20):
            R = rot(rng)
            c = np.array([0.0, 0.0, rng.uniform(-0.02, 0.09)])
            signs = [((i & 1) * 2 - 1, (i >> 1 & 1) * 2 - 1, (i >> 2 & 1) * 2 - 1) for i in range(8)]
            corners = [c + R @ (h * np.array(sg)) for sg in signs]
            expect = [v for v in corners if v[2] < margin]
            p, n, d = O.collide(dict(type=PLANE, pos=[0, 0, 0]), dict(type=BOX, pos=c, mat=R, size=h), margin=margin)
            np.testing.assert_allclose(d, [v[2] for v in expect], atol=1e-15)
            np.testing.assert_allclose(p, np.reshape([v - [0, 0, v[2] / 2] for v in expect], (-1, 3)), atol=1e-15)


# ------------------------------------------------------------------------------ sphere / capsule / box
def test_sphere_box_signed_distance():
    rng = np.random.default_rng(3)
    h = np.array([0.1, 0.05, 0.2])
    hits = 0
    for _ in range(600):
        R = rot(rng)
        c = rng.normal(size=3) * 0.1
        s = c + rng.uniform(-0.25, 0.25, 3)
        r = 0.05
        p, n, d = O.collide(dict(type=SPHERE, pos=s, size=[r]), dict(type=BOX, pos=c, mat=R, size=h), margin=0.0)
        sd = signed_point_box(s, c, R, h) - r
        assert (len(d) > 0) == (sd < 0)
        if len(d):
            hits += 1
            np.testing.assert_allclose(d[0], sd, atol=1e-12)
            assert abs(np.linalg.norm(n[0]) - 1) < 1e-12
            # the sphere witness is the sphere point deepest towards the box
            np.testing.assert_allclose(p[0] - 0.5 * d[0] * n[0], s + r * n[0], atol=1e-12)
    assert hits > 50


def brute_capsule_box(cap_c, cap_R, r, half, c, R, h):
    """Minimum over the segment of the signed point-box distance (a convex function of the
    segment parameter: the signed distance to a convex set is convex), by ternary search."""
    f = lambda t: signed_point_box(cap_c + t * half * cap_R[:, 2], c, R, h)  # noqa: E731
    lo, hi = -1.0, 1.0
    for _ in range(200):
        m1, m2 = lo + (hi - lo) / 3, hi - (hi - lo) / 3
        if f(m1) <= f(m2):
            hi = m2
        else:
            lo = m1
    return min(f(0.5 * (lo + hi)), f(-1.0), f(1.0)) - r


def test_capsule_box_depth_against_sampling():
    rng = np.random.default_rng(4)
    h = np.array([0.1, 0.06, 0.15])
    hits = 0
    for _ in range(120):
        R, Rc = rot(rng), rot(rng)
        c = np.zeros(3)
        cc = rng.uniform(-0.25, 0.25, 3)
        r, half = 0.03, 0.08
        p, n, d = O.collide(dict(type=CAPSULE, pos=cc, mat=Rc, size=[r, half]),
                            dict(type=BOX, pos=c, mat=R, size=h))
        ref = brute_capsule_box(cc, Rc, r, half, c, R, h)
        if abs(ref) < 1e-4:
            continue                      # grazing: sampling resolution
        assert (len(d) > 0) == (ref < 0)
        if len(d):
            hits += 1
            # sphere contacts sit on segment points: never deeper than the deepest segment point,
            # and exact while the segment itself stays outside the box
            assert d.min() >= ref - 1e-12
            if ref > -r:
                assert abs(d.min() - ref) < 1e-12
            for k in range(len(d)):
                assert abs(np.linalg.norm(n[k]) - 1) < 1e-12
    assert hits > 20


def test_capsule_capsule_segment_distance():
    rng = np.random.default_rng(5)
    hits = 0
    for _ in range(200):
        R1, R2 = rot(rng), rot(rng)
        c1, c2 = np.zeros(3), rng.uniform(-0.12, 0.12, 3)
        r1, r2, h1, h2 = 0.03, 0.02, 0.1, 0.07
        p, n, d = O.collide(dict(type=CAPSULE, pos=c1, mat=R1, size=[r1, h1]),
                            dict(type=CAPSULE, pos=c2, mat=R2, size=[r2, h2]))
        a = seg_points(c1, R1, h1, 801)
        b = seg_points(c2, R2, h2, 801)
        dd = np.sqrt(((a[:, None, :] - b[None, :, :]) ** 2).sum(-1)).min() - r1 - r2
        if abs(dd) < 1e-3:
            continue
        assert (len(d) > 0) == (dd < 0)
        if len(d):
            hits += 1
            assert abs(d.min() - dd) < 5e-4
            # normal points from capsule 1 to capsule 2
            w1 = p[0] - 0.5 * d[0] * n[0]
            assert np.dot(n[0], w1 - c1) > -1e-12 or np.linalg.norm(w1 - c1) < r1 + h1
    assert hits > 30


def test_capsule_capsule_parallel_two_contacts():
    R = np.eye(3)
    p, n, d = O.collide(dict(type=CAPSULE, pos=[0, 0, 0], mat=R, size=[0.03, 0.1]),
                        dict(type=CAPSULE, pos=[0.05, 0, 0.02], mat=R, size=[0.03, 0.1]))
    assert len(d) == 2
    np.testing.assert_allclose(d, [-0.01, -0.01], atol=1e-15)
    np.testing.assert_allclose(n, [[1, 0, 0], [1, 0, 0]], atol=1e-15)
    np.testing.assert_allclose(sorted(p[:, 2]), [-0.08, 0.1], atol=1e-15)


# ------------------------------------------------------------------------------ box-box
def test_boxbox_face_contacts_and_separation():
    size = np.ones((2, 3))
    mat = np.tile(np.eye(3), (2, 1, 1))
    for z, margin, depth in ((1.9, 0.0, -0.1), (2.01, 0.02, 0.01), (2.1, 0.02, None)):
        g1, g2 = boxes(size, [[0, 0, 0], [0, 0, z]], mat)
        p, n, d = O.collide(g1, g2, margin=margin)
        if depth is None:
            assert len(d) == 0
            continue
        assert len(np.unique(np.round(p, 12), axis=0)) == 4
        np.testing.assert_allclose(d, depth, atol=1e-14)
        np.testing.assert_allclose(n, np.tile([0, 0, 1], (4, 1)), atol=1e-15)


def test_boxbox_task5_book_contact():
    f = json.loads((GOLDEN / 'boxbox_task5.json').read_text())
    p, n, d = O.collide(*boxes(f['size'], f['pos'], f['mat']), margin=f['margin'])
    assert len(d) == 4
    assert d.min() > -2e-7 and d.max() <= 0
    np.testing.assert_allclose(d.min(), -f['physical_overlap'], rtol=1e-6)
    assert box_witnesses_ok(p, n, d, f['size'], f['pos'], f['mat'], 1e-12)


def test_boxbox_task5_rotations_swaps_scales():
    f = json.loads((GOLDEN / 'boxbox_task5.json').read_text())
    rng = np.random.RandomState(13)
    for scale in (1e-3, 1.0, 1e3):
        for swap in (False, True):
            for _ in range(6):
                q = rng.normal(size=4)
                Q = quat2mat(q / np.linalg.norm(q))
                size = np.asarray(f['size']) * scale
                pos = np.asarray(f['pos']) @ Q.T * scale
                mat = Q @ np.asarray(f['mat'])
                if swap:
                    size, pos, mat = size[::-1], pos[::-1], mat[::-1]
                p, n, d = O.collide(*boxes(size, pos, mat))
                assert len(d) > 0
                assert d.min() > -2e-7 * scale
                assert d.max() <= 1e-12 * scale


def test_boxbox_outside_candidates_fit_margin():
    f = json.loads((GOLDEN / 'boxbox_task5.json').read_text())
    for margin in (0.01, 2.0):
        p, n, d = O.collide(*boxes(f['size'], f['pos'], f['mat']), margin=margin)
        assert len(d) >= 4
        assert d.min() > -2e-7 and d.max() <= margin


def test_boxbox_first_incident_vertex_on_reference_face():
    rows = [np.array([float(x) for x in row]) for row in csv.reader((GOLDEN / 'boxbox_first_face_vertex.csv').open())]
    size, pos, mat = rows[0].reshape(2, 3), rows[1].reshape(2, 3), rows[2].reshape(2, 3, 3)
    for swap in (False, True):
        s, q, r = (a[::-1] if swap else a for a in (size, pos, mat))
        p, n, d = O.collide(*boxes(s, q, r))
        assert len(d) == 4
        for k in range(2):
            local = (p - q[k]) @ r[k]
            assert np.max(np.abs(local) - s[k]) <= 16 * np.finfo(np.float32).eps


def test_boxbox_edge_projection_witnesses():
    f = json.loads((GOLDEN / 'boxbox_edge_projection.json').read_text())
    p, n, d = O.collide(*boxes(f['size'], f['pos'], f['mat']))
    assert len(d) >= 1
    assert box_witnesses_ok(p, n, d, f['size'], f['pos'], f['mat'], 1e-10)
    np.testing.assert_allclose(-d.min(), sat_depth(f['size'], f['pos'], f['mat']), rtol=1e-9)


def test_boxbox_sat_face_tie_full_depth():
    rows = [np.array([float(x) for x in row]) for row in csv.reader((GOLDEN / 'boxbox_sat_face_tie.csv').open())]
    size = rows[0].reshape(2, 3)
    half_depth = rows[5][0]          # the native route's figure: half of the overlap
    for pos, mat in ((rows[1], rows[2]), (rows[3], rows[4])):
        pos, mat = pos.reshape(2, 3), mat.reshape(2, 3, 3)
        p, n, d = O.collide(*boxes(size, pos, mat))
        assert len(d) == 4
        np.testing.assert_allclose(d, 2 * half_depth, atol=1e-7)
        np.testing.assert_allclose(-d.min(), sat_depth(size, pos, mat), atol=1e-7)


def test_boxbox_random_pairs_against_sat():
    rng = np.random.RandomState(41)
    colliding = edges = 0
    for i in range(1000):
        size = 10 ** rng.uniform(-2, 0, (2, 3))
        mat = np.stack([rot(np.random.default_rng(rng.randint(1 << 30))) for _ in range(2)])
        pos = np.zeros((2, 3))
        pos[1] = rng.uniform(-1, 1, 3) * np.sum(size, axis=0)
        p, n, d = O.collide(*boxes(size, pos, mat))
        depth = sat_depth(size, pos, mat)
        if abs(depth) < 1e-9:
            continue
        assert (len(d) > 0) == (depth > 0), i
        if len(d):
            colliding += 1
            edges += len(d) == 1
            assert box_witnesses_ok(p, n, d, size, pos, mat, 1e-10), i
            np.testing.assert_allclose(np.linalg.norm(n, axis=1), 1, atol=1e-14)
            # a face is kept over a nearly aligned edge axis up to 5 % deeper
            # (mjwarp_box.cu:135-139), never deeper than that
            assert d.min() >= -depth / 0.95 - 1e-12, i
            assert d.max() <= 1e-12
    assert colliding > 300
    assert edges > 20


# ------------------------------------------------------------------------------ convex (GJK / EPA)
def make_hull(rng, n=20, semi=(0.05, 0.04, 0.03)):
    from scipy.spatial import ConvexHull
    p = rng.normal(size=(n, 3))
    p /= np.linalg.norm(p, axis=1, keepdims=True)
    p *= np.asarray(semi)
    v = p[ConvexHull(p).vertices]
    return v - v.mean(axis=0)


def polytope_overlap(A, B):
    """Exact penetration depth of two convex polytopes (world vertex arrays) by the separating-axis
    theorem over every face normal and every edge-edge cross product (< 0: separated)."""
    from scipy.spatial import ConvexHull

    def faces_edges(P):
        if len(P) == 2:
            return [], [P[1] - P[0]]
        h = ConvexHull(P)
        edges = [P[s[(i + 1) % 3]] - P[s[i]] for s in h.simplices for i in range(3)]
        return [e[:3] for e in h.equations], edges

    fa, ea = faces_edges(A)
    fb, eb = faces_edges(B)
    ea, eb = np.asarray(ea), np.asarray(eb)
    c = np.cross(ea[:, None, :], eb[None, :, :]).reshape(-1, 3)
    scale = (np.linalg.norm(ea, axis=1)[:, None] * np.linalg.norm(eb, axis=1)[None, :]).reshape(-1)
    ln = np.linalg.norm(c, axis=1)
    keep = ln > 1e-9 * scale
    axes = np.vstack([np.reshape(fa, (-1, 3)), np.reshape(fb, (-1, 3)), c[keep] / ln[keep, None]])
    pa, pb = A @ axes.T, B @ axes.T
    return float(np.min(np.minimum(pa.max(0) - pb.min(0), pb.max(0) - pa.min(0))))


def box_vertices(size, pos, R):
    s = np.array([[(i & 1) * 2 - 1, (i >> 1 & 1) * 2 - 1, (i >> 2 & 1) * 2 - 1] for i in range(8)], float)
    return (s * size) @ np.asarray(R).T + pos


@pytest.mark.parametrize('kind', ['hull-hull', 'box-hull'])
def test_epa_depth_equals_polytope_sat(kind):
    rng = np.random.default_rng(21 if kind == 'hull-hull' else 22)
    hits = misses = 0
    for _ in range(60):
        vb = make_hull(rng)
        R1, R2 = rot(rng), rot(rng)
        p2 = rng.uniform(-0.07, 0.07, 3)
        if kind == 'hull-hull':
            va = make_hull(rng)
            g1 = dict(type=7, pos=np.zeros(3), mat=R1, vert=va)
            A = va @ R1.T
        else:
            size = rng.uniform(0.02, 0.05, 3)
            g1 = dict(type=BOX, pos=np.zeros(3), mat=R1, size=size)
            A = box_vertices(size, np.zeros(3), R1)
        g2 = dict(type=7, pos=p2, mat=R2, vert=vb)
        depth = polytope_overlap(A, vb @ R2.T + p2)
        p, n, d = O.collide(g1, g2)
        if abs(depth) < 1e-6:
            continue
        assert (len(d) > 0) == (depth > 0)
        if len(d):
            hits += 1
            assert len(d) == 1
            assert abs(-d[0] - depth) < 2e-6, (d, depth)      # EPA stops at ccd tolerance 1e-6
            assert abs(np.linalg.norm(n[0]) - 1) < 1e-12
        else:
            misses += 1
    assert hits > 20 and misses > 5


def test_epa_horizon_overflow_flags_the_pair():
    """A horizon edge list beyond its capacity drops the pair's contact and sets
    MX_OVERFLOW_EPA_HORIZON (the reference's epa_horizon_overflow); at the normal capacity the same
    pairs give their contact and no flag."""
    rng = np.random.default_rng(31)
    flagged = 0
    try:
        for _ in range(20):
            va, vb = make_hull(rng), make_hull(rng)
            g1 = dict(type=7, pos=np.zeros(3), mat=rot(rng), vert=va)
            g2 = dict(type=7, pos=rng.uniform(-0.01, 0.01, 3), mat=rot(rng), vert=vb)   # deep overlap
            O.set_horizon_capacity(24)
            p, n, d = O.collide(g1, g2)
            assert len(d) == 1 and O.last_collide_flags() == 0
            O.set_horizon_capacity(3)
            p, n, d = O.collide(g1, g2)
            if O.last_collide_flags() & (1 << 8):
                assert len(d) == 0
                flagged += 1
            else:
                assert len(d) == 1
    finally:
        O.set_horizon_capacity(24)
    assert flagged > 10


def test_epa_capsule_hull_depth():
    """Capsule = segment + ball: where the segment itself penetrates the hull the depth is the
    segment-polytope SAT depth plus the radius (exact for the Minkowski sum)."""
    rng = np.random.default_rng(23)
    hits = 0
    for _ in range(80):
        vb = make_hull(rng, semi=(0.06, 0.05, 0.04))
        Rc, Rh = rot(rng), rot(rng)
        cc = rng.uniform(-0.03, 0.03, 3)
        r, half = 0.02, 0.05
        seg = np.array([cc - half * Rc[:, 2], cc + half * Rc[:, 2]])
        B = vb @ Rh.T
        seg_depth = polytope_overlap(seg, B)
        if seg_depth < 1e-4:
            continue
        p, n, d = O.collide(dict(type=CAPSULE, pos=cc, mat=Rc, size=[r, half]),
                            dict(type=7, pos=np.zeros(3), mat=Rh, vert=vb))
        assert len(d) == 1
        assert abs(-d[0] - (seg_depth + r)) < 2e-6, (d, seg_depth + r)
        hits += 1
    assert hits > 20


def test_convex_boxbox_route():
    """Box-box through GJK/EPA and the box manifold (the reference's route when no box has a
    margin): face contacts, the reference's book fixture, and existence / depth against SAT."""
    size = np.ones((2, 3))
    mat = np.tile(np.eye(3), (2, 1, 1))
    for z in (1.9, 1.99):
        p, n, d = O.collide(*boxes(size, [[0, 0, 0], [0, 0, z]], mat), boxbox='convex')
        assert len(d) == 4
        np.testing.assert_allclose(d, z - 2, atol=1e-12)
        np.testing.assert_allclose(np.abs(p[:, :2]), 1, atol=1e-12)
        np.testing.assert_allclose(p[:, 2], 1 + (z - 2) / 2, atol=1e-12)
    f = json.loads((GOLDEN / 'boxbox_task5.json').read_text())
    p, n, d = O.collide(*boxes(f['size'], f['pos'], f['mat']), boxbox='convex')
    assert len(d) == 4
    np.testing.assert_allclose(d, -f['physical_overlap'], rtol=1e-6)
    assert box_witnesses_ok(p, n, d, f['size'], f['pos'], f['mat'], 1e-12)
    rng = np.random.RandomState(41)
    single = 0
    for i in range(400):
        size = 10 ** rng.uniform(-2, 0, (2, 3))
        mat = np.stack([rot(np.random.default_rng(rng.randint(1 << 30))) for _ in range(2)])
        pos = np.zeros((2, 3))
        pos[1] = rng.uniform(-1, 1, 3) * np.sum(size, axis=0)
        p, n, d = O.collide(*boxes(size, pos, mat), boxbox='convex')
        depth = sat_depth(size, pos, mat)
        if abs(depth) < 1e-6:
            continue
        assert (len(d) > 0) == (depth > 0), i
        if len(d) == 1:
            single += 1
            assert abs(-d[0] - depth) < 2e-6 * max(1, depth), (i, d, depth)
    assert single > 50


# ---------------------------------------------------------------- hull against plane (plane_mesh)
def cube_vertices(h):
    return np.array([[x, y, z] for x in (-h, h) for y in (-h, h) for z in (-h, h)], float)


def test_plane_mesh_cube_resting_face():
    """A cube hull whose bottom face is 1 mm into the plane: the support corner and the other three
    corners of the bottom polygon, each at depth -1 mm, halfway between surface and corner."""
    h = 0.03
    plane = dict(type=PLANE, pos=np.zeros(3), mat=np.eye(3))
    cube = dict(type=7, pos=np.array([0.1, -0.2, h - 1e-3]), mat=np.eye(3), vert=cube_vertices(h))
    p, n, d = O.collide(plane, cube, margin=0.0)
    assert len(d) == 4
    np.testing.assert_allclose(d, -1e-3, atol=1e-15)
    np.testing.assert_allclose(n, np.tile([0, 0, 1.0], (4, 1)), atol=0)
    corners = sorted(map(tuple, np.round(p[:, :2], 12)))
    assert corners == sorted((0.1 + sx * h, -0.2 + sy * h) for sx in (-1, 1) for sy in (-1, 1))
    np.testing.assert_allclose(p[:, 2], -5e-4, atol=1e-15)


def test_plane_mesh_tilted_cube_corner_depths():
    """Tilted about x by theta, the bottom face stays the polygon most opposed to the plane normal:
    its four corners at the closed-form depths z_c - h cos(theta) +- h sin(theta)."""
    h, th, zc = 0.03, 0.2, 0.029
    R = np.array([[1, 0, 0], [0, np.cos(th), -np.sin(th)], [0, np.sin(th), np.cos(th)]])
    plane = dict(type=PLANE, pos=np.zeros(3), mat=np.eye(3))
    cube = dict(type=7, pos=np.array([0.0, 0.0, zc]), mat=R, vert=cube_vertices(h))
    p, n, d = O.collide(plane, cube, margin=0.05)
    assert len(d) == 4
    expect = sorted([zc - h * np.cos(th) - h * np.sin(th)] * 2 + [zc - h * np.cos(th) + h * np.sin(th)] * 2)
    np.testing.assert_allclose(sorted(d), expect, atol=1e-15)
    assert d[0] == min(d)                                   # the support corner comes first
    world = cube_vertices(h) @ R.T + cube['pos']
    for q, dist in zip(p, d):                               # every contact is a corner, shifted by d/2
        corner = q + 0.5 * dist * np.array([0, 0, 1.0])
        assert np.min(np.linalg.norm(world - corner, axis=1)) < 1e-15


def test_plane_mesh_random_hulls_properties():
    """Random hulls: contact 0 is the deepest vertex; the others are corners of one hull face that
    contains it, the face (from scipy's hull equations) whose outward normal is most opposed to the
    plane normal; at most four contacts, none above the hull's centre."""
    from scipy.spatial import ConvexHull
    rng = np.random.default_rng(31)
    checked = 0
    for _ in range(60):
        verts = make_hull(rng)
        R = rot(rng)
        pos = np.array([0.0, 0.0, rng.uniform(-0.01, 0.03)])
        plane = dict(type=PLANE, pos=np.zeros(3), mat=np.eye(3))
        p, n, d = O.collide(plane, dict(type=7, pos=pos, mat=R, vert=verts), margin=0.02)
        world = verts @ R.T + pos
        if not len(d):
            assert world[:, 2].min() >= 0.02
            continue
        checked += 1
        assert len(d) <= 4
        k0 = int(np.argmin(world[:, 2]))
        assert abs(d[0] - world[k0, 2]) < 1e-15
        hull = ConvexHull(verts)
        ln = R.T @ np.array([0, 0, 1.0])
        faces = [i for i, s in enumerate(hull.simplices) if k0 in s]
        best = min(faces, key=lambda i: hull.equations[i, :3] @ ln)
        nb, ob = hull.equations[best, :3], hull.equations[best, 3]
        for q, dist in zip(p, d):
            corner = q + 0.5 * dist * np.array([0, 0, 1.0])
            k = int(np.argmin(np.linalg.norm(world - corner, axis=1)))
            assert np.linalg.norm(world[k] - corner) < 1e-12
            assert abs(verts[k] @ nb + ob) < 1e-9            # on the chosen face's plane
            assert world[k, 2] <= pos[2] + 1e-15             # not above the centre
    assert checked > 30
