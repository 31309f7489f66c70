"""GPU parity of the MPR convex route (Options.mpr: MuJoCo 2.3.7 collision semantics, libccd's
ccdMPRPenetration, one contact per convex pair) against the CPU FP64 oracle.

The scene holds a static hull (the anvil) and, per world, a sphere, a capsule, a box and a hull
pressed into it from four sides at random orientations and depths of 0.5-4 mm (placed by bisection
on the oracle's GJK/EPA depth), so every convex family of the route occurs: sphere-hull, capsule-hull,
box-hull and hull-hull.  After the forward pass on both sides from the same FP32 state:

* contact counts and geom pairs exactly, positions and distances to 2e-5;
* normals to 1e-4 where a flat face or edge of the Minkowski difference decides them (box-hull,
  hull-hull), and to 5e-4 on a sphere's or capsule's round side, whose normal is the surface normal
  at the contact point (mjc_fixNormal): a position difference dp turns it by dp / radius; with
  geom margins (the variant with unequal margins and gaps, combined by the larger of each as MuJoCo
  2.3.7 does) every edge and vertex of the Minkowski difference is rounded with the pair's margin
  as radius, so the bar there is 2e-5 / margin;
* includemargin (margin - gap) to 1e-9;
* the constraint rows' kinds and efc_pos as for every other contact (2e-5).
"""
import math

import numpy as np
import pytest

from helpers import make_oracle
from libero_hip import scene as S
from libero_hip.model import Model, quat2mat
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ANVIL = np.array([2.0, 0.0, 0.5])


def _sphere(rng, radius):
    mass = rng.uniform(500.0, 1500.0) * 4.0 / 3.0 * math.pi * radius ** 3
    b = S.Body('ball', 0, mass=mass, inertia=(0.4 * mass * radius ** 2,) * 3)
    b.geoms.append(S.Geom(S.SPHERE, size=(radius, 0.0, 0.0)))
    b.joints.append(S.Joint(S.FREE))
    return b


def _geom_dict(geom, pos, mat):
    d = dict(type=geom.type, pos=pos, mat=mat, size=geom.size)
    if geom.vertices is not None:
        d['vert'] = np.asarray(geom.vertices, float)
    return d


def _press(anvil, geom, u, mat, depth, reach):
    """Distance along u from the anvil's centre at which the geoms penetrate by the given depth (the
    oracle's GJK/EPA: the minimum depth, continuous in the placement; MPR's depth along its own
    direction jumps to zero where the geoms come apart, a knife edge for a placement)."""
    lo, hi = 0.0, reach
    for _ in range(32):
        s = 0.5 * (lo + hi)
        dist = O.collide(_geom_dict(geom, ANVIL + s * u, mat), anvil)[2]
        if len(dist) and dist[0] < -depth:
            lo = s
        else:
            hi = s
    return hi


def mpr_scene(nworld, seed=0, margins=False):
    """margins: unequal nonzero geom margins and gaps on the anvil and the objects (MuJoCo 2.3.7
    combines them by the larger of each)."""
    rng = np.random.default_rng(seed)
    arm, actuators, osc, q_ready = S._arm()
    world = S._world(table=False)
    anvil_verts = S.make_hull(rng, 28, (0.07, 0.06, 0.05))
    world.geoms.append(S.Geom(S.MESH, pos=tuple(ANVIL), vertices=anvil_verts, contype=0, conaffinity=1))
    objects = [_sphere(rng, 0.025), S._object(rng, 'capsule', 'capsule')[0], S._object(rng, 'box', 'box')[0],
               S._object(rng, 'hull', 'hull')[0]]
    if margins:
        world.geoms[-1].margin, world.geoms[-1].gap = 0.003, 0.0005
        for k, body in enumerate(objects):
            body.geoms[0].margin, body.geoms[0].gap = 0.002 + 0.002 * k, 0.001 * (k % 2)
    opts = S.Options()
    opts.mpr, opts.nconmax = True, 32
    nq = 9 + 7 * len(objects)
    qpos = np.zeros((nworld, nq))
    anvil = dict(type=S.MESH, pos=ANVIL, mat=np.eye(3), vert=anvil_verts)
    reach = float(np.linalg.norm(anvil_verts, axis=1).max()) + 0.2
    for w in range(nworld):
        wrng = np.random.default_rng([seed, w])
        qpos[w, :7] = q_ready
        qpos[w, 7:9] = 0.02
        for k, body in enumerate(objects):
            az = k * math.pi / 2 + wrng.uniform(-0.35, 0.35)
            el = wrng.uniform(-0.35, 0.35)
            u = np.array([math.cos(el) * math.cos(az), math.cos(el) * math.sin(az), math.sin(el)])
            q = wrng.normal(size=4)
            q /= np.linalg.norm(q)
            s = _press(anvil, body.geoms[0], u, quat2mat(q), wrng.uniform(5e-4, 4e-3), reach)
            qpos[w, 9 + 7 * k:16 + 7 * k] = (*(ANVIL + s * u), *q)
    return S.Scene(name='mpr', bodies=[world] + arm + objects, actuators=actuators, options=opts, nworld=nworld,
                   substeps=25, osc=osc, init_qpos=qpos, init_qvel=np.zeros((nworld, 9 + 6 * len(objects))),
                   seed=seed)


@pytest.mark.parametrize('route,margins', [('workspace', False), ('lds', False), ('workspace', True)])
def test_mpr_contact_parity(gpu_available, route, margins):
    import torch
    from libero_hip import native
    nworld = 32
    sc = mpr_scene(nworld, seed=11, margins=margins)
    m = Model(sc)
    assert m.convex_mpr == 1 and m.boxbox_primitive == 1
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld, workspace=None if route == 'workspace' else False)
    om, od = make_oracle(m, nworld)
    qpos = sc.init_qpos.astype(np.float32).astype(np.float64)
    dd['qpos'].copy_(torch.from_numpy(qpos))
    dd['qvel'].zero_()
    dd['body_active'].fill_(1)
    dd['osc_gains'].copy_(torch.from_numpy(od['osc_gains']))
    dd['osc_q0'].copy_(torch.from_numpy(od['osc_q0']))
    od['qpos'][:] = qpos
    od['qvel'][:] = 0.0
    print('case mpr', route, 'ngeom', m.ngeom, flush=True)
    flags = native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL
    dd.forward(None, flags)
    od.forward(None, flags)
    torch.cuda.synchronize()
    g = {k: dd[k].double().cpu().numpy() for k in ('overflow', 'ncon', 'nefc', 'contact_geom', 'contact_pos',
                                                   'contact_dist', 'contact_frame', 'efc_type', 'efc_pos',
                                                   'contact_includemargin')}
    assert not g['overflow'].any() and not od['overflow'].any()
    np.testing.assert_array_equal(g['ncon'][:, 0], od['ncon'][:, 0])
    np.testing.assert_array_equal(g['nefc'][:, 0], od['nefc'][:, 0])
    gtype = m.arrays['geom_type']
    gmargin = m.arrays['geom_margin']
    families, worst = {}, {}
    for w in range(nworld):
        c, r = int(od['ncon'][w, 0]), int(od['nefc'][w, 0])
        gg, og = g['contact_geom'][w, :2 * c].reshape(-1, 2).astype(int), od['contact_geom'][w, :2 * c].reshape(-1, 2)
        np.testing.assert_array_equal(gg, og)
        for a, b in og:
            key = (int(gtype[a]), int(gtype[b]))
            families[key] = families.get(key, 0) + 1
        # one contact per pair on this route: the pairs identify the contacts
        assert len({(int(a), int(b)) for a, b in og}) == c
        errs = dict(pos=np.abs(g['contact_pos'][w, :3 * c] - od['contact_pos'][w, :3 * c]).reshape(-1, 3).max(axis=1),
                    dist=np.abs(g['contact_dist'][w, :c] - od['contact_dist'][w, :c]),
                    normal=np.abs(g['contact_frame'][w, :9 * c] - od['contact_frame'][w, :9 * c]).reshape(-1, 9)[:, :3]
                    .max(axis=1))
        round_side = np.isin(gtype[og[:, 0]], (S.SPHERE, S.CAPSULE))
        # with a margin the shapes are inflated by half of it each, so the Minkowski difference's
        # edges and vertices are rounded with the margin as radius: a position difference dp turns
        # the normal there by dp / margin
        margin = np.maximum(gmargin[og[:, 0]], gmargin[og[:, 1]])
        rounded = np.where(margin > 0, 2e-5 / np.maximum(margin, 1e-12), 0.0)
        bars = dict(pos=np.full(c, 2e-5), dist=np.full(c, 2e-5),
                    normal=np.maximum(np.where(round_side, 5e-4, 1e-4), rounded))
        for k in errs:
            worst[k] = max(worst.get(k, 0.0), float((errs[k] / bars[k]).max(initial=0.0)))
            assert (errs[k] <= bars[k]).all(), (w, k, errs[k], og)
        np.testing.assert_allclose(g['contact_includemargin'][w, :c], od['contact_includemargin'][w, :c], rtol=0,
                                   atol=1e-9)
        np.testing.assert_array_equal(np.sort(g['efc_type'][w, :r]), np.sort(od['efc_type'][w, :r]))
        np.testing.assert_allclose(np.sort(g['efc_pos'][w, :r]), np.sort(od['efc_pos'][w, :r]), rtol=0, atol=2e-5)
    print('mpr', route, 'margins', margins, 'families', families, 'worst error / bar', {k: '%.2f' % v for k, v in worst.items()})
    for key in ((S.SPHERE, S.MESH), (S.CAPSULE, S.MESH), (S.BOX, S.MESH), (S.MESH, S.MESH)):
        assert families.get(key, 0) >= nworld // 2, key
