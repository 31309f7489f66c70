"""stat_sums: per-world sums of constraint rows, contacts, Newton iterations and iterations x rows
over every substep computed since the caller cleared them (the counts a benchmark's
algorithmic-bytes figure averages).

* oracle (CPU): one 25-substep control step gives the sums of 25 one-substep launches from the same
  state, the counts read after each of them (the oracle is deterministic);
* device (marked gpu): the same against the kernel's own one-substep launches, and the row and
  contact sums equal the oracle's from the same FP32 state (identical contact sets, as the parity
  tests require).
"""
import numpy as np
import pytest

from helpers import make_oracle

STATE = ('qpos', 'qvel', 'qacc_warmstart', 'osc_goal_pos', 'osc_goal_rot', 'osc_gripper', 'ctrl', 'time')


def _oracle_settled(nworld=4, config='c3'):
    from libero_hip import scene as S
    from libero_hip.model import Model
    sc = S.make_scene(config, nworld, seed=4)
    m = Model(sc)
    om, od = make_oracle(m, nworld)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, 8 | 2)
    acts = S.make_actions(nworld, 3, seed=5)
    od['osc_action'][:] = acts[0]
    od.control_step(25, 1)
    return m, om, od, acts


def test_oracle_stat_sums_are_per_substep_sums():
    m, om, od, acts = _oracle_settled()
    start = {k: od[k].copy() for k in STATE}
    od['stat_sums'][:] = 0
    od['osc_action'][:] = acts[1]
    od.control_step(25, 1)
    sums = od['stat_sums'].copy()
    end = od['qpos'].copy()
    for k, v in start.items():
        od[k][:] = v
    per = np.zeros_like(sums)
    for s in range(25):
        od.control_step(1, 1 if s == 0 else 0)
        n, c, it = od['nefc'][:, 0], od['ncon'][:, 0], od['solver_niter'][:, 0]
        per += np.stack([n, c, it, it * n], 1)
    np.testing.assert_array_equal(od['qpos'], end)          # the same trajectory
    np.testing.assert_array_equal(sums, per)
    assert (sums[:, 0] > 0).all() and (sums[:, 3] >= sums[:, 0]).all()


@pytest.mark.gpu
def test_device_stat_sums(gpu_available):
    import torch
    from libero_hip import native
    m, om, od, acts = _oracle_settled(8)
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, 8)
    dd['body_active'].fill_(1)
    for k in STATE + ('osc_gains', 'osc_q0'):
        dd[k].copy_(torch.from_numpy(od[k]))
        od[k][:] = dd[k].double().cpu().numpy()
    start = {k: dd[k].clone() for k in STATE}
    for d in (dd, od):
        d['stat_sums'][:] = 0
    dd['osc_action'].copy_(torch.from_numpy(acts[1]))
    od['osc_action'][:] = acts[1]
    dd.control_step(25, native.FLAG_POLICY_FIRST)
    od.control_step(25, 1)
    torch.cuda.synchronize()
    sums = dd['stat_sums'].cpu().numpy()
    end = dd['qpos'].clone()
    np.testing.assert_array_equal(sums[:, :2], od['stat_sums'][:, :2])
    for k, v in start.items():
        dd[k].copy_(v)
    per = np.zeros_like(sums)
    for s in range(25):
        dd.control_step(1, native.FLAG_POLICY_FIRST if s == 0 else 0)
        n, c, it = (dd[k].cpu().numpy()[:, 0].astype(float) for k in ('nefc', 'ncon', 'solver_niter'))
        per += np.stack([n, c, it, it * n], 1)
    assert torch.equal(dd['qpos'], end)
    np.testing.assert_array_equal(sums, per)
