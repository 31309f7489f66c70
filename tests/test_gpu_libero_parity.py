"""GPU parity on LIBERO task scenes compiled from LIBERO's own asset MJCF and BDDL files.

The scenes are composed on the build machine by libero_hip.libero_task (arena, fixtures, objects,
the robot stand-in, LIBERO's options: elliptic cones, impratio 20, the medium's density and
viscosity) and loaded here from tests/golden/*.json (written by tests/golden/make_libero_scenes.py).
Each case settles the sampled initial state on the oracle for two control steps, then runs one
substep on the HIP kernel and on the FP64 oracle from the same state.

What is compared, and to what bar:

* contacts and rows exactly as for the benchmark scenes: counts, geom pairs, positions and
  distances (2e-5), frames (1e-4 or the FP32 bound of the convex route's normal), row types, ids
  and efc_pos; the state after the substep (qpos, qvel) and the smooth dynamics (qacc_smooth,
  qfrc_passive with the fluid forces) to 1e-4;
* constraint forces and accelerations (efc_force, qacc, qfrc_constraint) per world to
  max(1e-4, 4 s + 2 g): LIBERO's objects are light (grams) on stiff contacts (solref 0.001 clamped
  to 2 dt, solimp 0.998) with many contacts sharing each object's weight, so these outputs are
  ill-conditioned.  s is the oracle's own response to a perturbation of qpos and qvel by one FP32
  epsilon (1.2e-7) relative (the kernel's FP32 arithmetic perturbs every intermediate by a few of
  those), g the distance of
  the oracle's solution at the scene's solver tolerance (1e-6) from its converged solution (the
  Newton iterate stops anywhere in the flat directions of statically indeterminate contact sets, the
  kernel's as much as the oracle's, hence 2 g).
  Worlds whose contact or row count changes under that perturbation are contact-ambiguous and left
  out of the force comparison (at most a quarter of the worlds).
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import make_oracle, rel_err
from libero_hip import native, scene_io, scene as S
from libero_hip.model import Model
from test_gpu_contact_parity import STATE, _np, _settled, contact_rows, match_contacts

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / 'golden'
TASKS = ['libero_spatial_bowl_plate', 'libero_living_room_basket']
PERTURB = float(np.finfo(np.float32).eps)


def _world_forces(d, w, perm=None):
    """A world's efc_force rows: non-contact rows in order, then each contact's rows."""
    r, c = int(d['nefc'][w, 0]), int(d['ncon'][w, 0])
    typ, ids, f = d['efc_type'][w, :r], d['efc_id'][w, :r], d['efc_force'][w, :r]
    out = [f[typ < 5]]
    for i in range(c):
        out.append(f[contact_rows(typ, ids, i if perm is None else perm[i])])
    return np.concatenate(out) if r else np.zeros(0)


def _oracle_substep(sc, start, action, *, perturb=0.0, seed=0, tolerance=None):
    if tolerance is not None:
        sc.options.tolerance, sc.options.iterations = tolerance, 1000
    m = Model(sc)
    om, od = make_oracle(m, sc.nworld)
    for k, v in start.items():
        od[k][:] = v
    if perturb:
        rng = np.random.default_rng(seed)
        for k in ('qpos', 'qvel'):
            od[k][:] *= 1 + perturb * rng.standard_normal(od[k].shape)
    od['osc_action'][:] = action
    od.control_step(1, native.FLAG_POLICY_FIRST)
    return od


@pytest.mark.parametrize('task', TASKS)
def test_libero_task_one_substep_parity(gpu_available, task):
    import torch
    sc = scene_io.load(GOLDEN / (task + '.json'))
    assert sc.options.cone == S.ELLIPTIC and sc.options.density > 0 and sc.options.viscosity > 0
    nworld = sc.nworld
    m, dd, od, acts = _settled('libero', nworld, settle=2, seed=1, scene=sc)
    print('case libero', task, 'ngeom', m.ngeom, 'npair', m.npair, 'nv', m.nv, flush=True)
    start = {k: od[k].copy() for k in STATE}
    dd['osc_action'].copy_(torch.from_numpy(acts[0]))
    od['osc_action'][:] = acts[0]
    dd.control_step(1, native.FLAG_POLICY_FIRST)
    od.control_step(1, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    g = {k: _np(dd[k]) for k in ('overflow', 'ncon', 'nefc', 'contact_geom', 'contact_pos', 'contact_dist',
                                 'contact_frame', 'efc_type', 'efc_id', 'efc_force', 'efc_pos', 'qacc',
                                 'qfrc_constraint', 'qpos', 'qvel', 'qacc_smooth', 'qfrc_passive')}
    assert not g['overflow'].any() and not od['overflow'].any()
    pert = [_oracle_substep(scene_io.load(GOLDEN / (task + '.json')), start, acts[0], perturb=PERTURB, seed=s)
            for s in (1, 2)]
    conv = _oracle_substep(scene_io.load(GOLDEN / (task + '.json')), start, acts[0], tolerance=1e-13)
    for name in ('qpos', 'qvel', 'qacc_smooth', 'qfrc_passive'):
        assert rel_err(g[name], od[name]) < 1e-4, name
    ambiguous, worst, rows = [], {}, set()
    for w in range(nworld):
        c, r = int(od['ncon'][w, 0]), int(od['nefc'][w, 0])
        if any(p['ncon'][w, 0] != c or p['nefc'][w, 0] != r for p in pert) or conv['nefc'][w, 0] != r:
            ambiguous.append(w)
            continue
        assert g['ncon'][w, 0] == c and g['nefc'][w, 0] == r, w
        gg, og = g['contact_geom'][w, :2 * c].reshape(-1, 2), od['contact_geom'][w, :2 * c].reshape(-1, 2)
        np.testing.assert_array_equal(gg, og)
        gpos, opos = g['contact_pos'][w, :3 * c].reshape(-1, 3), od['contact_pos'][w, :3 * c].reshape(-1, 3)
        perm = match_contacts(gpos, gg, opos, og, c)
        np.testing.assert_allclose(gpos, opos[perm], rtol=0, atol=2e-5)
        odist = od['contact_dist'][w, :c][perm]
        np.testing.assert_allclose(g['contact_dist'][w, :c], odist, rtol=0, atol=2e-5)
        rel = np.linalg.norm(opos[perm] - od['geom_xpos'][w].reshape(-1, 3)[og[perm, 0]], axis=1)
        ftol = np.maximum(1e-4, 4 * np.finfo(np.float32).eps * rel / np.maximum(np.abs(odist), 1e-9))
        ferr = np.abs(g['contact_frame'][w, :9 * c].reshape(-1, 9) - od['contact_frame'][w, :9 * c].reshape(-1, 9)[perm])
        assert (ferr.max(axis=1) <= ftol).all(), w
        gt, ot = g['efc_type'][w, :r], od['efc_type'][w, :r]
        np.testing.assert_array_equal(np.sort(gt), np.sort(ot))
        rows |= set(int(t) for t in ot)
        # constraint forces and accelerations against the conditioning of this world
        of = _world_forces(od, w)
        s = max(max(rel_err(_world_forces(p, w), of, floor=1e-3) for p in pert),
                max(rel_err(p['qacc'][w], od['qacc'][w]) for p in pert))
        gap = max(rel_err(_world_forces(conv, w), of, floor=1e-3), rel_err(conv['qacc'][w], od['qacc'][w]))
        tol = max(1e-4, 4 * s + 2 * gap)
        errs = dict(efc_force=rel_err(_world_forces(g, w), _world_forces(od, w, perm), floor=1e-3),
                    qacc=rel_err(g['qacc'][w], od['qacc'][w]),
                    qfrc_constraint=rel_err(g['qfrc_constraint'][w], od['qfrc_constraint'][w]))
        for k, v in errs.items():
            worst[k] = max(worst.get(k, 0.0), v / tol)
            assert v <= tol, (w, k, v, 'tolerance', tol, 'sensitivity', s, 'solver gap', gap)
    print('libero', task, 'ambiguous worlds', ambiguous, 'worst error / tolerance',
          {k: '%.2f' % v for k, v in worst.items()}, 'row kinds', sorted(rows))
    assert len(ambiguous) <= nworld // 4
    assert 7 in rows                                      # elliptic contact rows


@pytest.mark.parametrize('task', TASKS)
def test_libero_task_rollout(gpu_available, task):
    """Four control steps (100 substeps) from the settled state: qpos drift against the oracle within
    the bound of the benchmark scenes' rollout test (tests/test_gpu_contact_parity.py)."""
    import torch
    sc = scene_io.load(GOLDEN / (task + '.json'))
    m, dd, od, acts = _settled('libero', sc.nworld, settle=2, seed=1, scene=sc)
    print('case libero rollout', task, flush=True)
    for k in range(4):
        dd['osc_action'].copy_(torch.from_numpy(acts[k]))
        od['osc_action'][:] = acts[k]
        dd.control_step(sc.substeps, native.FLAG_POLICY_FIRST)
        od.control_step(sc.substeps, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    assert not _np(dd['overflow']).any() and not od['overflow'].any()
    drift = np.abs(_np(dd['qpos']) - od['qpos']).max(axis=1)
    print('libero rollout', task, 'qpos drift per world: max %.2e median %.2e' % (drift.max(), np.median(drift)))
    assert np.isfinite(_np(dd['qpos'])).all()
    assert drift.max() < 5e-2
