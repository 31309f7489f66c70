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
* constraint forces and accelerations per world to max(1e-4, 4 s + 2 g), capped at 1e-3 for qacc
  and qfrc_constraint (the generalized constraint force J^T f, which drives the dynamics) and at
  1e-2 for efc_force.  LIBERO's objects are light (grams) on stiff contacts (solref 0.001 clamped
  to 2 dt, solimp 0.998) with several contacts sharing each object's weight, so these outputs are
  ill-conditioned.  s is the larger of two measured sensitivities to a one-ulp change of the FP32
  state: the oracle's (FP64 arithmetic; qpos and qvel scaled by 1 + eps32 N(0, 1), two draws) and
  the device's own (the same kernel on the state with random entries of qpos and qvel moved by one
  ulp, three draws), which includes the FP32 arithmetic's rounding.  The split of an object's load among its
  contacts (efc_force; J^T f does not depend on it) is determined only weakly, by the contacts'
  compliance: in the bowl-and-plate scene the device moves it by up to 3e-3 under a one-ulp
  change of its own input, so no FP32 route can hold efc_force to 1e-3 there, while J^T f stays
  within 4e-5.  At the scene's solver tolerance (1e-6) the Newton iterate stops anywhere in those
  flat directions, up to 1.6e-2 from the converged forces, so the compared substep runs both sides
  at a solver tolerance of 1e-10 (1000 iterations), where the FP32 iterate stops at its rounding
  floor and the oracle's converges; g is what remains of the oracle's distance from its fully
  converged (1e-13) solution.  Worlds whose contact or row count changes under the perturbation
  are contact-ambiguous and left out of the force comparison, at most one world in eight.  Each
  case prints per world the errors, s and g, then the largest bar, the worlds whose bar exceeds
  1e-4, the worst error over the bar and the worlds left out.
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import make_oracle, rel_err
from libero_hip import native, scene_io, scene as S
from libero_hip.model import Model
from test_gpu_contact_parity import STATE, _np, _settled, contact_rows, frame_tolerance, match_contacts

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / 'golden'
TASKS = ['libero_spatial_bowl_plate', 'libero_living_room_basket', 'libero_object_soup_basket', 'libero_goal_wine_rack',
         'libero_10_mugs_plates']
PERTURB = float(np.finfo(np.float32).eps)
TIGHT = 1e-10          # the compared substep's solver tolerance (both sides)
CAP = {'efc_force': 1e-2, 'qacc': 1e-3, 'qfrc_constraint': 1e-3}
LEGAL = (1 << 9) | (1 << 10)   # the solver's iteration-limit bits


def _world_forces(d, w, perm=None):
    """A world's efc_force rows: non-contact rows in order, then each contact's rows."""
    r, c = int(d['nefc'][w, 0]), int(d['ncon'][w, 0])
    typ, ids, f = d['efc_type'][w, :r], d['efc_id'][w, :r], d['efc_force'][w, :r]
    out = [f[typ < 5]]
    for i in range(c):
        out.append(f[contact_rows(typ, ids, i if perm is None else perm[i])])
    return np.concatenate(out) if r else np.zeros(0)


def _device_substep(dmodel, start, action, seed=5):
    """The kernel's substep from the start state with random entries of qpos and qvel moved by one
    FP32 ulp (the device's own sensitivity to its input rounding)."""
    import torch
    d = native.DeviceData(dmodel, start['qpos'].shape[0])
    d['body_active'].fill_(1)
    rng = np.random.default_rng(seed)
    for k, v in start.items():
        if k in ('qpos', 'qvel'):
            v32 = v.astype(np.float32)
            v = np.where(rng.random(v32.shape) < 0.5, np.nextafter(v32, np.float32(np.inf)), v32).astype(np.float64)
        d[k].copy_(torch.from_numpy(v))
    d['osc_action'].copy_(torch.from_numpy(action))
    d.control_step(1, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    return {k: _np(d[k]) for k in ('ncon', 'nefc', 'efc_type', 'efc_id', 'efc_force', 'qacc', 'qfrc_constraint')}


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
    sc.options.tolerance, sc.options.iterations = TIGHT, 1000
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
    assert not (g['overflow'] & ~LEGAL).any() and not (od['overflow'] & ~LEGAL).any()
    pert = [_oracle_substep(scene_io.load(GOLDEN / (task + '.json')), start, acts[0], perturb=PERTURB, seed=s,
                            tolerance=TIGHT) for s in (1, 2)]
    conv = _oracle_substep(scene_io.load(GOLDEN / (task + '.json')), start, acts[0], tolerance=1e-13)
    devs = [_device_substep(dd.dmodel, start, acts[0], seed=k) for k in (5, 6, 7)]
    for name in ('qpos', 'qvel', 'qacc_smooth', 'qfrc_passive'):
        assert rel_err(g[name], od[name]) < 1e-4, name
    ambiguous, worst, largest, rows, tols, frames, failures = [], {}, {}, set(), [], [0, 0], []
    for w in range(nworld):
        c, r = int(od['ncon'][w, 0]), int(od['nefc'][w, 0])
        if any(p['ncon'][w, 0] != c or p['nefc'][w, 0] != r for p in pert + devs) or conv['nefc'][w, 0] != r:
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
        ftol = frame_tolerance(m, od, w, og[perm], opos[perm], odist)
        ferr = np.abs(g['contact_frame'][w, :9 * c].reshape(-1, 9)
                      - od['contact_frame'][w, :9 * c].reshape(-1, 9)[perm]).max(axis=1)
        assert (ferr <= ftol).all(), w
        frames[0] += c
        frames[1] += int((ferr > 1e-4).sum())
        gt, ot = g['efc_type'][w, :r], od['efc_type'][w, :r]
        np.testing.assert_array_equal(np.sort(gt), np.sort(ot))
        rows |= set(int(t) for t in ot)
        # constraint forces and accelerations against the conditioning of this world
        of = _world_forces(od, w)
        gf = _world_forces(g, w)
        sens = {'efc_force': max([rel_err(_world_forces(p, w), of, floor=1e-3) for p in pert]
                                 + [rel_err(_world_forces(d, w), gf, floor=1e-3) for d in devs])}
        for k in ('qacc', 'qfrc_constraint'):
            sens[k] = max([rel_err(p[k][w], od[k][w]) for p in pert] + [rel_err(d[k][w], g[k][w]) for d in devs])
        gaps = {'efc_force': rel_err(_world_forces(conv, w), of, floor=1e-3)}
        for k in ('qacc', 'qfrc_constraint'):
            gaps[k] = rel_err(conv[k][w], od[k][w])
        bars = {k: min(CAP[k], max(1e-4, 4 * sens[k] + 2 * gaps[k])) for k in sens}
        tol = max(bars.values())
        tols.append(tol)
        s, gap = max(sens.values()), max(gaps.values())
        errs = dict(efc_force=rel_err(_world_forces(g, w), _world_forces(od, w, perm), floor=1e-3),
                    qacc=rel_err(g['qacc'][w], od['qacc'][w]),
                    qfrc_constraint=rel_err(g['qfrc_constraint'][w], od['qfrc_constraint'][w]))
        for k, v in errs.items():
            worst[k] = max(worst.get(k, 0.0), v / bars[k])
            largest[k] = max(largest.get(k, 0.0), v)
            if v > bars[k]:
                failures.append((w, k, v, 'bar', bars[k], 'sensitivity', sens[k], 'solver gap', gaps[k]))
        print('  world %2d ' % w + ' | '.join('%s %.1e (s %.1e g %.1e bar %.1e)' % (k, errs[k], sens[k], gaps[k], bars[k])
                                              for k in errs))
    print('libero', task, 'worlds', nworld, 'left out (contact-ambiguous)', ambiguous,
          'bar: largest %.2e, median %.2e, above 1e-4 in %d worlds' % (max(tols), float(np.median(tols)),
                                                                        int((np.array(tols) > 1e-4).sum())),
          'worst error / bar', {k: '%.2f' % v for k, v in worst.items()},
          'largest error', {k: '%.1e' % v for k, v in largest.items()},
          'frames: %d contacts, %d above 1e-4' % tuple(frames), 'row kinds', sorted(rows))
    assert not failures, failures
    assert len(ambiguous) <= nworld // 8
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
