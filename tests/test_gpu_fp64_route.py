"""The FP64 route (MX_FLAG_FP64: the physics computed in double, each world's working set in LDS)
against the CPU FP64 oracle.

The oracle gets the FP32-rounded model (OracleModel(fp32_model=True): the values the device's model
arena holds) and the device's FP32 state, so the two compute from identical inputs in double; what
remains is summation order, the Newton solver's stopping point and the rounding of the outputs to
the FP32 fields of MxData (relative 6e-8).  C1 (elliptic cones) and C3 (boxes, capsules, hulls,
pyramidal cones) from an oracle-settled state with resting contacts:

* one substep: identical contact sets and row types; contact positions, distances and frames
  within 1e-6; efc_force, qacc, qacc_smooth, qfrc_constraint within 1e-6 relative (max-abs error
  over max-abs reference); qpos and qvel within 1e-6 relative.  The FP32 route's errors on the same
  step are printed beside them and must be larger (the route computes in double);
* C1, one 25-substep control step: qpos, qvel within 1e-5 relative, printed with the FP32 route's;
* C3, 25 substeps each restarted from the device's state: world-substeps agree to 1e-6 in qacc
  except where a convex-route contact (a hull resting face-down on the table) has no unique EPA
  witness point: there the two EPAs, rounding differently, pick different points on the touching
  faces (same depth within 1e-5 m, same rows and states), and the contact Jacobian moves with the
  point; such departures are counted (at most one world-substep in ten);
* the environment at precision "fp64" runs this route (precision reported as fp64) and refuses a
  model whose FP64 working set exceeds the LDS of a workgroup (C4).
"""
import numpy as np
import pytest

from helpers import make_oracle, rel_err
from test_gpu_contact_parity import STATE, _np, match_contacts

pytestmark = pytest.mark.gpu


def _settled64(config, nworld, settle=2, seed=0):
    import torch
    from libero_hip import scene as S, native
    from libero_hip.model import Model
    sc = S.make_scene(config, nworld, seed=seed)
    m = Model(sc)
    om, od = make_oracle(m, nworld, fp32_model=True)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    acts = S.make_actions(nworld, settle + 2, seed=seed + 2)
    for k in range(settle):
        od['osc_action'][:] = acts[k]
        od.control_step(25, native.FLAG_POLICY_FIRST)
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld)
    for name in STATE:
        dd[name].copy_(torch.from_numpy(od[name]))
        od[name][:] = _np(dd[name])
    if m.body_active is None:
        dd['body_active'].fill_(1)
    else:
        dd['body_active'].copy_(torch.from_numpy(m.body_active))
    return m, dd, od, acts[settle:]


def _device_runs(dd, action, substeps):
    """The same launch through the FP32 and the FP64 route from the same device state; the fields
    each run leaves, by route."""
    import torch
    from libero_hip import native
    start = {k: dd[k].clone() for k in STATE}
    keep = ('qpos', 'qvel', 'qacc', 'qacc_smooth', 'qfrc_constraint', 'ncon', 'nefc', 'contact_geom', 'contact_pos',
            'contact_dist', 'contact_frame', 'efc_type', 'efc_id', 'efc_force', 'overflow', 'solver_niter')
    out = {}
    for route, flag in (('fp32', 0), ('fp64', native.FLAG_FP64)):
        for k in STATE:
            dd[k].copy_(start[k])
        dd['osc_action'].copy_(torch.from_numpy(action))
        dd.control_step(substeps, native.FLAG_POLICY_FIRST | flag)
        torch.cuda.synchronize()
        out[route] = {k: _np(dd[k]).copy() for k in keep}
    return out


def _contact_errors(g, od, nworld):
    """Largest contact position, distance and frame errors and the efc_force error (matched
    contacts); asserts identical contact sets and row types."""
    ncon, nefc = g['ncon'][:, 0], g['nefc'][:, 0]
    np.testing.assert_array_equal(ncon, od['ncon'][:, 0])
    np.testing.assert_array_equal(nefc, od['nefc'][:, 0])
    err = dict(pos=0.0, dist=0.0, frame=0.0, efc_force=0.0)
    for w in range(nworld):
        c, r = int(ncon[w]), int(nefc[w])
        ggeom = g['contact_geom'][w, :2 * c].reshape(-1, 2)
        ogeom = od['contact_geom'][w, :2 * c].reshape(-1, 2)
        np.testing.assert_array_equal(ggeom, ogeom)
        gpos = g['contact_pos'][w, :3 * c].reshape(-1, 3)
        opos = od['contact_pos'][w, :3 * c].reshape(-1, 3)
        perm = match_contacts(gpos, ggeom, opos, ogeom, c)
        err['pos'] = max(err['pos'], float(np.abs(gpos - opos[perm]).max(initial=0)))
        err['dist'] = max(err['dist'], float(np.abs(g['contact_dist'][w, :c] - od['contact_dist'][w, :c][perm]).max(initial=0)))
        gf = g['contact_frame'][w, :9 * c].reshape(-1, 9)
        of = od['contact_frame'][w, :9 * c].reshape(-1, 9)[perm]
        err['frame'] = max(err['frame'], float(np.abs(gf - of).max(initial=0)))
        gt, gi, gfo = g['efc_type'][w, :r], g['efc_id'][w, :r], g['efc_force'][w, :r]
        ot, oi, ofo = od['efc_type'][w, :r], od['efc_id'][w, :r], od['efc_force'][w, :r]
        np.testing.assert_array_equal(gt[gt < 5], ot[ot < 5])
        grows, orows = [gfo[gt < 5]], [ofo[ot < 5]]
        for i in range(c):
            gr = np.where((gi == i) & (gt >= 5))[0]
            orr = np.where((oi == perm[i]) & (ot >= 5))[0]
            np.testing.assert_array_equal(gt[gr], ot[orr])
            grows.append(gfo[gr])
            orows.append(ofo[orr])
        if r:
            err['efc_force'] = max(err['efc_force'], rel_err(np.concatenate(grows), np.concatenate(orows), floor=1e-3))
    return err


@pytest.mark.parametrize('config,nworld', [('c1', 16), ('c3', 32)])
def test_fp64_route_one_substep(gpu_available, config, nworld):
    from libero_hip import native
    m, dd, od, acts = _settled64(config, nworld)
    print('case', config, nworld, 'fp64 lds bytes', dd.dmodel.lds_bytes_fp64(), flush=True)
    runs = _device_runs(dd, acts[0], 1)
    od['osc_action'][:] = acts[0]
    od.control_step(1, native.FLAG_POLICY_FIRST)
    errs = {}
    for route, g in runs.items():
        assert not g['overflow'].any()
        e = _contact_errors(g, od, nworld)
        for name in ('qacc', 'qacc_smooth', 'qfrc_constraint', 'qvel', 'qpos'):
            e[name] = rel_err(g[name], od[name])
        errs[route] = e
        print(config, route, {k: '%.2e' % v for k, v in e.items()}, 'niter', g['solver_niter'][:4, 0],
              od['solver_niter'][:4, 0], flush=True)
    assert od['ncon'].max() > 0
    for k, v in errs['fp64'].items():
        assert v < 1e-6, (k, v)
    # the route computes in double: its largest error is far below the FP32 route's
    assert max(errs['fp64'].values()) < 0.1 * max(errs['fp32'].values())


def test_fp64_route_control_step_c1(gpu_available):
    """C1: one 25-substep control step on both routes; the FP64 route within 1e-5 relative."""
    from libero_hip import native
    m, dd, od, acts = _settled64('c1', 16, seed=3)
    runs = _device_runs(dd, acts[0], 25)
    od['osc_action'][:] = acts[0]
    od.control_step(25, native.FLAG_POLICY_FIRST)
    for route, g in runs.items():
        assert not (g['overflow'] & ~((1 << 9) | (1 << 10))).any()
        e = {name: rel_err(g[name], od[name]) for name in ('qpos', 'qvel')}
        print('c1', route, 'control step', {k: '%.2e' % v for k, v in e.items()}, flush=True)
        if route == 'fp64':
            for k, v in e.items():
                assert v < 1e-5, (k, v)


def test_fp64_route_substeps_c3(gpu_available):
    """C3: 25 substeps, both sides restarted from the device's state before each (so that one
    departure does not carry into the next).  A world-substep departs when its qacc differs by more
    than 1e-6 relative; every departure must come from a convex-route contact (a hull on the table
    or a box pair) whose EPA witness point is not unique: same geom pairs, row types and states,
    the contact's distance within 1e-5 m, its position elsewhere on the touching faces.  Departures
    are counted and printed; all other world-substeps agree to the FP32 rounding of the outputs."""
    import torch
    from libero_hip import native
    from libero_hip import scene as S
    m, dd, od, acts = _settled64('c3', 32, seed=3)
    gtype = m.arrays['geom_type']
    dd['osc_action'].copy_(torch.from_numpy(acts[0]))
    od['osc_action'][:] = acts[0]
    departures, worst_other = [], 0.0
    for s in range(25):
        flags = native.FLAG_POLICY_FIRST if s == 0 else 0
        dd.control_step(1, flags | native.FLAG_FP64)
        od.control_step(1, flags)
        torch.cuda.synchronize()
        g = {k: _np(dd[k]) for k in ('qacc', 'ncon', 'nefc', 'efc_type', 'efc_state', 'contact_geom', 'contact_pos',
                                       'contact_dist', 'overflow')}
        assert not (g['overflow'] & ~((1 << 9) | (1 << 10))).any()
        np.testing.assert_array_equal(g['ncon'], od['ncon'])
        np.testing.assert_array_equal(g['nefc'], od['nefc'])
        for w in range(dd.nworld):
            o = od['qacc'][w]
            err = np.abs(g['qacc'][w] - o).max() / max(np.abs(o).max(), 1e-6)
            if err <= 1e-6:
                worst_other = max(worst_other, err)
                continue
            c, r = int(g['ncon'][w, 0]), int(g['nefc'][w, 0])
            np.testing.assert_array_equal(g['efc_type'][w, :r], od['efc_type'][w, :r])
            np.testing.assert_array_equal(g['efc_state'][w, :r], od['efc_state'][w, :r])
            gg = g['contact_geom'][w, :2 * c].reshape(-1, 2)
            np.testing.assert_array_equal(gg, od['contact_geom'][w, :2 * c].reshape(-1, 2))
            np.testing.assert_allclose(g['contact_dist'][w, :c], od['contact_dist'][w, :c], rtol=0, atol=1e-5)
            moved = np.where(np.abs(g['contact_pos'][w, :3 * c].reshape(-1, 3)
                                    - od['contact_pos'][w, :3 * c].reshape(-1, 3)).max(axis=1) > 1e-6)[0]
            assert len(moved) > 0, (s, w, err)
            for k in moved:
                t1, t2 = gtype[gg[k]]
                assert t2 == S.MESH or (t1 == S.BOX and t2 == S.BOX and m.boxbox_primitive == 0), (s, w, k, t1, t2)
            departures.append((s, w, float(err), [tuple(int(x) for x in gg[k]) for k in moved]))
        for k in STATE:
            od[k][:] = _np(dd[k])
    print('c3 fp64 substeps: %d of %d world-substeps depart (EPA witness points), others within %.2e'
          % (len(departures), 25 * dd.nworld, worst_other), departures, flush=True)
    assert worst_other <= 1e-6
    assert len(departures) <= 25 * dd.nworld // 10


def test_fp64_environment(gpu_available):
    """HipBatchEnv at precision fp64 steps on this route; C4's FP64 working set does not fit LDS."""
    from libero_hip import layout
    from libero_hip.environment import HipBatchEnv
    env = HipBatchEnv('c3', 4, precision='fp64', graph=False)
    try:
        obs = env.reset()
        acts = np.zeros((4, 7))
        acts[:, 0] = 0.5
        for _ in range(2):
            obs, reward, done, info = env.step(acts)
        diag = env.diagnostics()
        assert diag['precision'] == 'fp64' and diag['lds_bytes_per_world'] <= layout.LDS_BUDGET
        assert np.isfinite(env.get_sim_state()).all()
        assert all(n == 50 for n in diag['actual_integration_count'])
    finally:
        env.close()
    with pytest.raises(ValueError, match='fp64'):
        HipBatchEnv('c4', 2, precision='fp64', graph=False)
