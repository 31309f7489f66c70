"""GPU parity of the contact path (collision, constraint rows, Newton) against the CPU FP64 oracle.

Both implementations start a control step from the same settled state: the oracle first runs a
few seeded control steps so that objects rest on the table and touch each other, the state is
copied to the device and the oracle's copy is rounded to the device's FP32 values (so both start
from bit-identical inputs), then both take one substep (and, for the drift report, several control
steps) through their C ABIs.

Tolerances (FP32 device vs FP64 oracle, one substep):
* contact set: identical count and geom pairs per world; within one geom pair the contacts are
  compared as a set (matched by position), since near-ties between equally deep faces may order
  the same points differently in FP32 and FP64 (the reference's own order is that of its atomic
  append); positions and distances within 2e-5 m; frames within 1e-4, or, for a convex-route pair
  where larger, the FP32 rounding bound 4 eps32 |p - o| / |dist| of that route's normal, which is
  the normalized difference of a manifold point pair |dist| apart (mjwarp_convex_collision.cuh:74)
  computed at positions relative to o, the centre of the pair's geom with the smaller bounding
  radius (where the kernel translates the pair), so a resting box-box contact 4e-5 m deep carries a
  few 1e-4 of FP32 noise in its normal; the contacts admitted above 1e-4 are counted and printed;
* constraint rows: identical count; per matched contact identical row types, efc_force within 1e-4
  relative (max-abs error over max-abs reference, per world), efc_pos within 2e-5 m (contact rows)
  and 1e-6 (joint limits: the distance at build time); qfrc_constraint and qacc within 1e-4
  relative;
* rollout drift over four control steps: reported, bounded loosely as a sanity check.
"""
import numpy as np
import pytest

from helpers import rel_err, make_oracle

pytestmark = pytest.mark.gpu

STATE = ('qpos', 'qvel', 'qacc_warmstart', 'osc_goal_pos', 'osc_goal_rot', 'osc_gripper', 'osc_gains',
         'osc_q0', 'ctrl', 'time')



def _np(t):
    import torch
    return t.cpu().numpy() if t.dtype == torch.int32 else t.double().cpu().numpy()


def match_contacts(gpos, ggeom, opos, ogeom, n):
    """perm[i] = oracle contact matched to device contact i (same geom pair, nearest position)."""
    perm = -np.ones(n, int)
    used = np.zeros(n, bool)
    for i in range(n):
        cand = [j for j in range(n) if not used[j] and tuple(ogeom[j]) == tuple(ggeom[i])]
        assert cand, 'device contact %d has no oracle counterpart' % i
        j = min(cand, key=lambda j: np.sum((opos[j] - gpos[i]) ** 2))
        perm[i] = j
        used[j] = True
    return perm


def frame_tolerance(m, od, w, og, opos, odist):
    """Per-contact frame tolerance of world w (oracle geom pairs og, positions opos, distances odist):
    1e-4, and for convex-route pairs (hull pairs; box-box unless the primitive routine is selected)
    the larger of that and 4 eps32 |p - o| / |dist|, o the centre of the geom with the smaller
    bounding radius."""
    from libero_hip import scene as S
    gtype, rbound = m.arrays['geom_type'], m.arrays['geom_rbound']
    xpos = od['geom_xpos'][w].reshape(-1, 3)
    t1, t2 = gtype[og[:, 0]], gtype[og[:, 1]]
    convex = (t1 != S.PLANE) & ((t2 == S.MESH) | ((t1 == S.BOX) & (t2 == S.BOX) & (m.boxbox_primitive == 0)))
    small = np.where(rbound[og[:, 1]] < rbound[og[:, 0]], og[:, 1], og[:, 0])
    rel = np.linalg.norm(opos - xpos[small], axis=1)
    bound = 4 * np.finfo(np.float32).eps * rel / np.maximum(np.abs(odist), 1e-9)
    return np.where(convex, np.maximum(1e-4, bound), 1e-4)


def contact_rows(typ, cid, c):
    return np.where((cid == c) & (typ >= 5))[0]


def _settled(config, nworld, settle=3, seed=0, workspace=None, scene=None):
    """Oracle-settled state of `config` (or of the given `scene`) copied to a device batch; the
    oracle keeps the device's FP32 values of it."""
    import torch
    from libero_hip import scene as S, native
    from libero_hip.model import Model
    sc = scene if scene is not None else S.make_scene('c3' if config == 'c3floor' else config, nworld, seed=seed)
    if config == 'c3floor':   # the two hulls moved off the table onto the ground plane (plane_mesh)
        for k, y in ((4, -0.2), (5, 0.2)):
            radius = float(np.linalg.norm(sc.bodies[-6 + k].geoms[0].vertices, axis=1).max())
            sc.init_qpos[:, 9 + 7 * k:12 + 7 * k] = (1.3, y, radius + 0.002)
    m = Model(sc)
    om, od = make_oracle(m, nworld)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    acts = S.make_actions(nworld, settle + 4, seed=seed + 2)
    for k in range(settle):
        od['osc_action'][:] = acts[k]
        od.control_step(25, native.FLAG_POLICY_FIRST)
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld, workspace=workspace)
    for name in STATE:
        dd[name].copy_(torch.from_numpy(od[name]))
        od[name][:] = _np(dd[name])          # the same inputs: the device's FP32 values
    if m.body_active is None:
        dd['body_active'].fill_(1)
    else:
        dd['body_active'].copy_(torch.from_numpy(m.body_active))
    return m, dd, od, acts[settle:]


# route 'workspace' (the default for models with constraint rows) keeps each world's working set in
# a device-memory slab of MxData.workspace; 'lds' allocates no workspace, so the working set stays in
# LDS (c4 exceeds LDS and has the workspace route only)
@pytest.mark.parametrize('config,nworld,route', [('c1', 16, 'workspace'), ('c3', 64, 'workspace'),
                                                 ('c3floor', 32, 'workspace'), ('c3floor', 32, 'lds'),
                                                 ('c5', 32, 'workspace'), ('c4', 16, 'workspace'),
                                                 ('c1', 16, 'lds'), ('c3', 64, 'lds'), ('c5', 32, 'lds')])
def test_one_substep_contact_parity(gpu_available, config, nworld, route):
    m, dd, od, acts = _settled(config, nworld, workspace=None if route == 'workspace' else False)
    assert (dd['workspace'].shape[1] > 1) == (route == 'workspace')
    print('case', config, nworld, route, 'lds bytes', dd.dmodel.lds_bytes(), flush=True)
    compare_one_substep(m, dd, od, acts[0], '%s %s' % (config, route))


def compare_one_substep(m, dd, od, action, label):
    """One policy substep on both sides from the same state; asserts the module's tolerances and
    returns the contacts' (geom type 1, geom type 2) families and the row types that occurred."""
    import torch
    from libero_hip import native
    nworld = dd.nworld
    acts = [action]
    dd['osc_action'].copy_(torch.from_numpy(acts[0]))
    od['osc_action'][:] = acts[0]
    dd.control_step(1, native.FLAG_POLICY_FIRST)
    od.control_step(1, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    assert not _np(dd['overflow']).any() and not od['overflow'].any()
    ncon, nefc = _np(dd['ncon'])[:, 0], _np(dd['nefc'])[:, 0]
    np.testing.assert_array_equal(ncon, od['ncon'][:, 0])
    np.testing.assert_array_equal(nefc, od['nefc'][:, 0])
    # every world of a homogeneous batch touches something; heterogeneous ones may hold no objects
    assert (ncon.min() if m.body_active is None else ncon.max()) > 0
    worst = {}
    frames = [0, 0, 0.0]        # contacts, contacts whose frame differs by more than 1e-4, largest
    for w in range(nworld):
        c, r = int(ncon[w]), int(nefc[w])
        ggeom = _np(dd['contact_geom'])[w, :2 * c].reshape(-1, 2)
        ogeom = od['contact_geom'][w, :2 * c].reshape(-1, 2)
        np.testing.assert_array_equal(ggeom, ogeom)             # same pairs in the same order
        gpos = _np(dd['contact_pos'])[w, :3 * c].reshape(-1, 3)
        opos = od['contact_pos'][w, :3 * c].reshape(-1, 3)
        perm = match_contacts(gpos, ggeom, opos, ogeom, c)
        np.testing.assert_array_equal(_np(dd['contact_dim'])[w, :c], od['contact_dim'][w, :c][perm])
        np.testing.assert_allclose(gpos, opos[perm], rtol=0, atol=2e-5)
        np.testing.assert_allclose(_np(dd['contact_dist'])[w, :c], od['contact_dist'][w, :c][perm], rtol=0,
                                   atol=2e-5)
        # frames: 1e-4, or the FP32 cancellation bound of the convex route's normal
        odist = od['contact_dist'][w, :c][perm]
        ftol = frame_tolerance(m, od, w, ogeom[perm], opos[perm], odist)
        ferr = np.abs(_np(dd['contact_frame'])[w, :9 * c].reshape(-1, 9)
                      - od['contact_frame'][w, :9 * c].reshape(-1, 9)[perm]).max(axis=1)
        assert (ferr <= ftol).all(), (w, ferr.max(), ftol[np.argmax(ferr - ftol)])
        frames[0] += c
        frames[1] += int((ferr > 1e-4).sum())
        frames[2] = max(frames[2], float(ferr.max(initial=0.0)))
        gt, gi, gf = _np(dd['efc_type'])[w, :r], _np(dd['efc_id'])[w, :r], _np(dd['efc_force'])[w, :r]
        ot, oi, of = od['efc_type'][w, :r], od['efc_id'][w, :r], od['efc_force'][w, :r]
        gp_, op_ = _np(dd['efc_pos'])[w, :r], od['efc_pos'][w, :r]
        # rows that are not contact rows (dof friction, joint limits) keep their order
        np.testing.assert_array_equal(gt[gt < 5], ot[ot < 5])
        np.testing.assert_array_equal(gi[gt < 5], oi[ot < 5])
        np.testing.assert_allclose(gp_[gt < 5], op_[ot < 5], rtol=0, atol=1e-6)
        g_rows = [gf[gt < 5]]
        o_rows = [of[ot < 5]]
        for i in range(c):
            gr, orow = contact_rows(gt, gi, i), contact_rows(ot, oi, perm[i])
            np.testing.assert_array_equal(gt[gr], ot[orow])
            np.testing.assert_allclose(gp_[gr], op_[orow], rtol=0, atol=2e-5)
            g_rows.append(gf[gr])
            o_rows.append(of[orow])
        if r:
            g_all, o_all = np.concatenate(g_rows), np.concatenate(o_rows)
            worst['efc_force'] = max(worst.get('efc_force', 0), rel_err(g_all, o_all, floor=1e-3))
    for name in ('qacc', 'qfrc_constraint', 'qacc_smooth', 'qvel', 'qpos'):
        worst[name] = rel_err(_np(dd[name]), od[name])
    print(label, {k: '%.2e' % v for k, v in worst.items()},
          'niter gpu/oracle', _np(dd['solver_niter'])[:4, 0], od['solver_niter'][:4, 0])
    print(label, 'frames: %d contacts, %d above 1e-4 (within the convex-route bound), largest %.2e'
          % tuple(frames))
    for k, v in worst.items():
        assert v < 1e-4, (k, v)
    gtype = m.arrays['geom_type']
    families = {}
    for w in range(nworld):
        for g1, g2 in od['contact_geom'][w, :2 * int(ncon[w])].reshape(-1, 2):
            key = (int(gtype[g1]), int(gtype[g2]))
            families[key] = families.get(key, 0) + 1
    rows = set(int(t) for w in range(nworld) for t in od['efc_type'][w, :int(nefc[w])])
    return families, rows


@pytest.mark.parametrize('config,nworld', [('c1', 8), ('c3', 16), ('c5', 16), ('c4', 4)])
def test_contact_rollout_drift(gpu_available, config, nworld):
    """Four 25-substep control steps with contacts: qpos drift against the oracle is reported."""
    import torch
    from libero_hip import native
    m, dd, od, acts = _settled(config, nworld, settle=2, seed=1)
    print('case', config, nworld, flush=True)
    for k in range(4):
        dd['osc_action'].copy_(torch.from_numpy(acts[k]))
        od['osc_action'][:] = acts[k]
        dd.control_step(25, native.FLAG_POLICY_FIRST)
        od.control_step(25, native.FLAG_POLICY_FIRST)
        torch.cuda.synchronize()
        per_world = np.abs(_np(dd['qpos']) - od['qpos']).max(axis=1)
        drift = per_world.max()
        print('%s control %d qpos drift max %.3e median %.3e ncon %s / %s'
              % (config, k, drift, np.median(per_world), _np(dd['ncon'])[:4, 0], od['ncon'][:4, 0]))
    assert np.isfinite(_np(dd['qpos'])).all()
    assert drift < 5e-2


def test_workspace_route_matches_lds_route(gpu_available):
    """The same control step through both routes from the same state: the same arithmetic except
    for summation orders (the line search holds one row per lane in registers on the workspace
    route, eight on the LDS route), so the two agree to FP32 rounding."""
    import torch
    from libero_hip import native
    m, dd, od, acts = _settled('c3', 32, settle=2, seed=5)
    dd['osc_action'].copy_(torch.from_numpy(acts[0]))
    start = {name: dd[name].clone() for name in STATE}
    out = {}
    for route, flag in (('lds', native.FLAG_LDS), ('workspace', 0)):
        for name in STATE:
            dd[name].copy_(start[name])
        dd.control_step(1, native.FLAG_POLICY_FIRST | flag)
        torch.cuda.synchronize()
        out[route] = {k: _np(dd[k]).copy() for k in ('qacc', 'qpos', 'qvel', 'efc_force', 'ncon', 'nefc')}
    np.testing.assert_array_equal(out['lds']['ncon'], out['workspace']['ncon'])
    np.testing.assert_array_equal(out['lds']['nefc'], out['workspace']['nefc'])
    for k in ('qacc', 'qpos', 'qvel', 'efc_force'):
        e = rel_err(out['workspace'][k], out['lds'][k], floor=1e-3)
        print('lds vs workspace', k, '%.2e' % e)
        assert e < 1e-5, (k, e)
