"""GPU parity of the observation sampler and of the environment's masked reset.

* the device sampler against its CPU restatement (oracle/observations.py: robosuite formulas in
  FP64, FP32 clocks): the device steps one substep per launch (mx_control_step_observed with one
  substep) and the CPU sampler is fed the fields the device published after each substep, so the
  comparison isolates the sampler from the FP32-vs-FP64 physics.  Observed values within 1e-5, the
  sampling state (present, sampled, events, elapsed) identical;
* the same two control steps as 25-substep launches (sampling inside the launch after every
  substep) give bit-identical observations and physics, and sampling leaves the physics
  bit-identical to mx_control_step.
* HipBatchEnv.reset(id=[...]) / set_init_state(..., id=[...]) restore the selected worlds and leave
  every other world's state, warm start, controller goal and observations bit-identical (the
  reference holds unselected worlds, gpu/host/backends/cuda_fp32/environment.py:143-212).
* HipBatchEnv._snapshot, the predicate boundary, equals direct reads of the device state after a
  step and after a masked reset, and feeds the predicate callback whose results step() returns.
"""
import numpy as np
import pytest

from test_gpu_contact_parity import _settled, _np

pytestmark = pytest.mark.gpu


def _fields(d):
    return {k: (d[k] if isinstance(d[k], np.ndarray) else _np(d[k])) for k in ('qpos', 'qvel', 'site_xpos', 'xpos',
                                                                             'xquat')}


STATE = ('qpos', 'qvel', 'qacc_warmstart', 'ctrl', 'time', 'osc_goal_pos', 'osc_goal_rot', 'osc_gripper', 'osc_gains',
         'osc_q0', 'osc_tau', 'body_active')


@pytest.mark.parametrize('config,nworld', [('c3', 16), ('c1', 8)])
def test_observations_match_the_cpu_sampler(gpu_available, config, nworld):
    import torch
    from libero_hip import native, observations as OB
    from oracle import observations as OO
    m, dd, od, acts = _settled(config, nworld, settle=2, seed=3)
    plan = OB.default_plan(m)
    print('case observations', config, nworld, 'specs', len(plan.specs), 'width', plan.width, flush=True)
    batches = []
    for _ in range(3):      # split launches with the CPU sampler, fused launches, no sampling
        d = native.DeviceData(dd.dmodel, nworld)
        for name in STATE:
            d[name].copy_(dd[name])
        d.forward(None, native.FLAG_NO_CONTROL)           # publish the fields
        batches.append(d)
    split, fused, plain = batches
    devs = [OB.DeviceObservations(plan, m, nworld) for _ in range(2)]
    cpu = OO.Sampler(plan, nworld)
    for dev, d in zip(devs, (split, fused)):               # the forced first sample, as after a reset
        dev.reset(d)
        dev.sample(d, force=True)
    cpu.reset(range(nworld))
    cpu.sample(_fields(split), m.opt.timestep, range(nworld), force=True)
    for k in range(2):
        for d in batches:
            d['osc_action'].copy_(torch.from_numpy(acts[k]))
        for s in range(25):
            devs[0].control_step(split, 1, native.FLAG_POLICY_FIRST if s == 0 else 0)
            cpu.sample(_fields(split), m.opt.timestep, range(nworld))
        devs[1].control_step(fused, 25, native.FLAG_POLICY_FIRST)
        plain.control_step(25, native.FLAG_POLICY_FIRST)
        torch.cuda.synchronize()
        got = devs[0].observed.cpu().numpy()
        err = np.abs(got - cpu.observed).max()
        print('control %d observed max abs err %.2e, events %d' % (k, err, int(cpu.events.sum())))
        assert err < 1e-5, err
        for name in ('present', 'sampled', 'events', 'elapsed'):
            np.testing.assert_array_equal(devs[0].state[name].cpu().numpy(), getattr(cpu, name), err_msg=name)
        assert cpu.present.all()
        for name in devs[0].state:
            assert torch.equal(devs[0].state[name], devs[1].state[name]), name
        for name in ('qpos', 'qvel', 'qacc', 'qacc_warmstart', 'efc_force', 'xpos', 'site_xpos', 'ncon'):
            assert torch.equal(split[name], fused[name]), name
            assert torch.equal(fused[name], plain[name]), name


def test_masked_reset_holds_other_worlds(gpu_available):
    import torch
    from libero_hip.environment import HipBatchEnv
    from libero_hip import scene as S
    env = HipBatchEnv('c3', 16, scene_seed=2)
    try:
        obs0 = env.reset()
        assert obs0['robot0_proprio-state'].shape[0] == 16
        acts = S.make_actions(16, 3, seed=4)
        for k in range(2):
            obs, rewards, successes, infos = env.step(acts[k])
        d = env.data
        names = ('qpos', 'qvel', 'qacc_warmstart', 'ctrl', 'time', 'osc_goal_pos', 'osc_goal_rot', 'osc_gripper',
                 'nstep', 'xpos', 'qacc')
        before = {n: d[n].clone() for n in names}
        obs_before = env.observer.observed.clone()
        sel = [5, 11]
        obs_r = env.reset(id=sel)
        keep = [w for w in range(16) if w not in sel]
        for n in names:
            assert torch.equal(d[n][keep], before[n][keep]), n
        assert torch.equal(env.observer.observed[keep], obs_before[keep])
        # the reset worlds are back at their initial states, their observations sampled afresh
        init = env.initial_states[np.asarray(sel) % len(env.initial_states)]
        np.testing.assert_allclose(_np(d['qpos'])[sel], init[:, 1:1 + env.model.nq], atol=1e-6)
        assert (_np(d['qvel'])[sel] == 0).all()
        qa = env.model.arrays['osc_qposadr']
        np.testing.assert_allclose(obs_r['robot0_joint_pos'], init[:, 1 + qa], atol=1e-6)
        np.testing.assert_allclose(obs_r['robot0_joint_pos_cos'], np.cos(init[:, 1 + qa]), atol=1e-6)
        # set_init_state on other worlds: the rest (the just-reset ones included) stay put
        before = {n: d[n].clone() for n in names}
        states = env.get_sim_state()[[0, 3]]
        states[:, 1:8] += 0.05
        env.set_init_state(states, id=[2, 9])
        keep = [w for w in range(16) if w not in (2, 9)]
        for n in names:
            assert torch.equal(d[n][keep], before[n][keep]), n
        np.testing.assert_allclose(_np(d['qpos'])[[2, 9]], states[:, 1:1 + env.model.nq], atol=1e-6)
        obs, rewards, successes, infos = env.step(acts[2])
        assert np.isfinite(obs['robot0_proprio-state']).all() and len(infos) == 16
    finally:
        env.close()


def test_snapshot_boundary(gpu_available):
    """HipBatchEnv._snapshot (the reference's predicate boundary, gpu/host/backends/cuda_fp32/
    environment.py:215-254) equals direct reads of the device state after a step and after a masked
    reset (contacts of the other worlds kept, those of the reset worlds recomputed); the predicate
    callback receives it with the world ids and its rewards and successes come back from step()."""
    from libero_hip.environment import HipBatchEnv, GOAL_FIELDS
    from libero_hip import scene as S
    calls = []

    def predicates(snapshot, ids):
        calls.append((sorted(snapshot), list(ids)))
        z = np.array([snapshot['body_xpos'][w, -1, 2] for w in ids])
        return z, np.array([snapshot['ncon'][w] > 0 for w in ids])

    names = GOAL_FIELDS + ('xpos', 'xquat', 'xmat', 'geom_xpos', 'geom_xmat', 'subtree_com', 'time', 'qvel', 'qacc',
                           'qacc_warmstart', 'ctrl', 'act', 'qfrc_applied', 'xfrc_applied', 'qfrc_bias', 'qfrc_smooth',
                           'qfrc_constraint', 'cfrc_ext', 'cfrc_int', 'sensordata')
    env = HipBatchEnv('c3', 8, scene_seed=3, predicates=predicates)
    try:
        m, d = env.model, env.data
        acts = S.make_actions(8, 3, seed=8)
        for k in range(2):
            obs, rewards, successes, infos = env.step(acts[k])
        assert calls[-1] == (sorted(GOAL_FIELDS), list(range(8)))
        snap = env._snapshot(names)

        def direct(name, shape):
            return _np(d[name])[:, :int(np.prod(shape))].reshape((8,) + shape)

        np.testing.assert_array_equal(snap['body_xpos'], direct('xpos', (m.nbody, 3)))
        np.testing.assert_array_equal(snap['xquat'], direct('xquat', (m.nbody, 4)))
        np.testing.assert_array_equal(snap['site_xmat'], direct('site_xmat', (m.nsite, 9)))
        np.testing.assert_array_equal(snap['geom_xpos'], direct('geom_xpos', (m.ngeom, 3)))
        np.testing.assert_array_equal(snap['qpos'], direct('qpos', (m.nq,)))
        np.testing.assert_array_equal(snap['cfrc_ext'], direct('cfrc_ext', (m.nbody, 6)))
        assert snap['time'].shape == (8,) and snap['act'].shape == (8, 0)
        np.testing.assert_array_equal(rewards, snap['body_xpos'][:, -1, 2])
        ncon = _np(d['ncon'])[:, 0].astype(int)
        np.testing.assert_array_equal(snap['ncon'], ncon)
        assert (ncon > 0).all() and successes.all()
        geoms = _np(d['contact_geom'])
        for w in range(8):
            pairs = np.stack([snap['contact'][w]['geom1'], snap['contact'][w]['geom2']], 1)
            np.testing.assert_array_equal(pairs, geoms[w, :2 * ncon[w]].reshape(-1, 2))
        # a masked reset: the other worlds' boundary fields unchanged, the reset ones read afresh
        before = env._snapshot(GOAL_FIELDS)
        env.reset(id=[2, 5])
        assert calls[-1][1] == [2, 5]
        after = env._snapshot(GOAL_FIELDS)
        keep = [w for w in range(8) if w not in (2, 5)]
        for name in ('qpos', 'body_xpos', 'body_xquat', 'site_xpos', 'site_xmat', 'ncon'):
            np.testing.assert_array_equal(after[name][keep], before[name][keep])
        for w in keep:
            for k in ('geom1', 'geom2'):
                np.testing.assert_array_equal(after['contact'][w][k], before['contact'][w][k])
        ncon = _np(d['ncon'])[:, 0].astype(int)
        geoms = _np(d['contact_geom'])
        for w in (2, 5):
            assert after['ncon'][w] == ncon[w]
            np.testing.assert_array_equal(after['contact'][w]['geom1'], geoms[w, 0:2 * ncon[w]:2])
        np.testing.assert_array_equal(after['qpos'][[2, 5]], direct('qpos', (m.nq,))[[2, 5]])
        with pytest.raises(KeyError, match='cam_xpos'):
            env._snapshot(('qpos', 'cam_xpos'))
    finally:
        env.close()
