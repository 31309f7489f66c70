"""GPU parity of the smooth-dynamics control step (config 2 shape) against the CPU FP64 oracle.

Both implementations start from the same state (seeded qpos/qvel, bootstrapped OSC goal) and
run through the C ABI (libmx_physics.so) and the oracle library respectively.

Tolerances:
* qacc, qacc_smooth, qfrc_bias, M, frames after one substep: 1e-4 relative (max-abs error over
  max-abs reference, per world), FP32 physics vs FP64 oracle;
* OSC torques: 1e-9 relative in the FP64 section, checked by feeding the controller inputs the GPU
  gathered (its FP32 M, J, q, qdot, bias, EE pose/velocity) into the oracle's FP64 OSC;
* short-rollout qpos drift: reported (printed), bounded loosely only as a sanity check.
"""
import numpy as np
import pytest

from helpers import rel_err, seeded_state, make_oracle

pytestmark = pytest.mark.gpu


def six_joint_scene(nworld, seed=0):
    """The config 2 scene with the wrist's last hinge removed: a 6-joint arm (link 7 welded to link
    6), six torque motors and the two finger servos."""
    from libero_hip import scene as S
    sc = S.make_scene('c2', nworld, seed=seed)
    link7 = next(b for b in sc.bodies if b.name == 'link7')
    link7.joints = []
    acts = [a for a in sc.actuators if a.joint != 6]
    for a in acts:
        if a.joint > 6:
            a.joint -= 1
    sc.actuators = acts
    sc.osc = dict(sc.osc, arm_joints=list(range(6)), actuators=list(range(8)), q0=np.asarray(sc.osc['q0'])[:6])
    sc.init_qpos = np.delete(sc.init_qpos, 6, axis=1)
    sc.init_qvel = np.delete(sc.init_qvel, 6, axis=1)
    return sc


def _pair(config, nworld, seed=0, scene=None):
    import torch
    from libero_hip import scene as S, native
    from libero_hip.model import Model
    sc = scene if scene is not None else S.make_scene(config, nworld, seed=seed)
    m = Model(sc)
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld)
    om, od = make_oracle(m, nworld)
    qpos, qvel = seeded_state(m, nworld, seed + 1)
    dd['qpos'].copy_(torch.from_numpy(qpos))
    dd['qvel'].copy_(torch.from_numpy(qvel))
    dd['osc_gains'].copy_(torch.from_numpy(od['osc_gains']))
    dd['osc_q0'].copy_(torch.from_numpy(od['osc_q0']))
    dd['body_active'].fill_(1)
    od['qpos'][:] = qpos
    od['qvel'][:] = qvel
    flags = native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL
    dd.forward(None, flags)
    od.forward(None, flags)
    torch.cuda.synchronize()
    return m, dd, od


def _np(t):
    return t.double().cpu().numpy()


def test_forward_parity(gpu_available):
    m, dd, od = _pair('c2', 64)
    for name in ('xpos', 'xmat', 'site_xpos', 'site_xmat', 'subtree_com', 'M', 'qfrc_bias',
                 'qfrc_passive', 'qacc_smooth'):
        e = rel_err(_np(dd[name]), od[name])
        print(name, e)
        assert e < 1e-4, (name, e)
    assert np.allclose(_np(dd['osc_goal_pos']), od['osc_goal_pos'], atol=1e-5)


@pytest.mark.parametrize('arm', ['7-joint', '6-joint'])
def test_one_substep_parity(gpu_available, arm):
    import torch
    from libero_hip import scene as S, native
    m, dd, od = _pair('c2', 64, scene=six_joint_scene(64) if arm == '6-joint' else None)
    print('case one substep', arm, 'osc joints', m.osc_ndof, flush=True)
    assert m.osc_ndof == (6 if arm == '6-joint' else 7)
    actions = S.make_actions(64, 1, seed=3)[0]
    dd['osc_action'].copy_(torch.from_numpy(actions))
    od['osc_action'][:] = actions
    gp0, gr0, gg0 = od['osc_goal_pos'].copy(), od['osc_goal_rot'].copy(), od['osc_gripper'].copy()
    dd.control_step(1, native.FLAG_POLICY_FIRST)
    od.control_step(1, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    assert not _np(dd['osc_error']).any()
    for name in ('qacc', 'qacc_smooth', 'qfrc_bias', 'qfrc_actuator', 'M', 'ctrl', 'qvel', 'qpos'):
        e = rel_err(_np(dd[name]), od[name])
        print(name, e)
        assert e < 1e-4, (name, e)
    # FP64 section: the oracle OSC on the GPU's own FP32 inputs
    from oracle import oracle as O
    ranges = m.arrays['actuator_ctrlrange'][m.arrays['osc_actuator']].reshape(-1)
    worst = 0.0
    for w in range(64):
        inp = dict(mass=_np(dd['osc_mass'])[w], jac=_np(dd['osc_jac'])[w], q=_np(dd['osc_q'])[w],
                   qvel=_np(dd['osc_qvel'])[w], bias=_np(dd['osc_bias'])[w], ee_pos=_np(dd['osc_ee_pos'])[w],
                   ee_rot=_np(dd['osc_ee_rot'])[w], ee_vel=_np(dd['osc_ee_vel'])[w])
        err, tau, ctrl, rank, gp, gr, gg = O.osc(inp, actions[w], od['osc_gains'][w], od['osc_q0'][w], ranges,
                                                 gp0[w], gr0[w], gg0[w], policy=True)
        assert err == 0
        worst = max(worst, rel_err(_np(dd['osc_tau'])[w], tau))
        assert np.allclose(_np(dd['osc_goal_pos'])[w], gp, rtol=0, atol=1e-12)
        assert np.allclose(_np(dd['osc_goal_rot'])[w], gr, rtol=0, atol=1e-12)
        assert np.array_equal(_np(dd['osc_rank'])[w], rank)
    print('osc tau rel', worst)
    assert worst < 1e-9


def test_rollout_drift(gpu_available):
    """25-substep control steps with seeded actions: qpos drift vs the FP64 oracle is reported."""
    import torch
    from libero_hip import scene as S, native
    m, dd, od = _pair('c2', 32)
    acts = S.make_actions(32, 4, seed=5)
    for c in range(4):
        dd['osc_action'].copy_(torch.from_numpy(acts[c]))
        od['osc_action'][:] = acts[c]
        dd.control_step(25, native.FLAG_POLICY_FIRST)
        od.control_step(25, native.FLAG_POLICY_FIRST)
        torch.cuda.synchronize()
        per_world = np.abs(_np(dd['qpos']) - od['qpos']).max(axis=1)
        drift = per_world.max()
        print('c2 control %d qpos drift max %.3e median %.3e' % (c, drift, np.median(per_world)))
    assert np.isfinite(drift) and drift < 5e-2
    assert (_np(dd['nstep']) == 100).all()


def test_env_api(gpu_available):
    from libero_hip.environment import HipBatchEnv
    from libero_hip import scene as S
    with HipBatchEnv('c2', 16, graph=True) as env:
        state0 = env.get_sim_state()
        assert state0.shape == (16, 1 + env.model.nq + env.model.nv)
        acts = S.make_actions(16, 3, seed=1)
        for a in acts:
            obs, r, s, info = env.step(a)
        assert obs['robot0_eef_pos'].shape == (16, 3)
        st = env.get_sim_state()
        assert np.allclose(st[:, 0], 3 * 25 * 0.002, atol=1e-4)
        env.set_init_state(state0[:4], id=[0, 1, 2, 3])
        st2 = env.get_sim_state()
        assert np.allclose(st2[:4, 1:], state0[:4, 1:], atol=1e-6)
        diag = env.diagnostics()
        assert diag['physics_engine'] == 'hip_mi355x'
        env.reset(id=[5])


def test_graph_replay_matches_eager(gpu_available):
    """A captured control step replayed several times equals eager launches bit for bit."""
    import torch
    from libero_hip.environment import HipBatchEnv
    from libero_hip import scene as S
    acts = S.make_actions(8, 3, seed=9)
    out = []
    for graph in (False, True):
        with HipBatchEnv('c2', 8, graph=graph) as env:
            for a in acts:
                env.step(a)
            out.append(env.get_sim_state())
    assert np.array_equal(out[0], out[1])


@pytest.mark.parametrize('config,nworld', [('c2', 64), ('c5', 64), ('c2-6-joint', 64)])
def test_standalone_osc_kernel(gpu_available, config, nworld):
    """mx_osc (the FP64 controller alone, from the inputs the last substep published) against the
    oracle's FP64 OSC on the same inputs, policy step with new actions: tau within 1e-9 relative,
    goal within 1e-12, ranks exact; and a non-policy call reproduces the in-kernel controller's tau
    of that substep bit for bit."""
    import torch
    from libero_hip import scene as S, native
    from oracle import oracle as O
    m, dd, od = _pair(config, nworld, scene=six_joint_scene(nworld) if config == 'c2-6-joint' else None)
    if m.body_active is not None:
        dd['body_active'].copy_(torch.from_numpy(m.body_active))
    acts = S.make_actions(nworld, 2, seed=7)
    dd['osc_action'].copy_(torch.from_numpy(acts[0]))
    dd.control_step(25, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    tau_kernel = dd['osc_tau'].clone()
    grip = _np(dd['osc_gripper']).copy()
    dd.osc(0)                                  # the last substep's controller once more
    torch.cuda.synchronize()
    assert torch.equal(dd['osc_tau'], tau_kernel)
    sgn = np.sign(acts[0][:, 6])
    np.testing.assert_array_equal(_np(dd['osc_gripper']), np.clip(grip + np.float32(0.01) * np.stack([-sgn, sgn], 1),
                                                                  -1, 1))
    inputs = {k: _np(dd[k]).copy() for k in ('osc_mass', 'osc_jac', 'osc_q', 'osc_qvel', 'osc_bias', 'osc_ee_pos',
                                             'osc_ee_rot', 'osc_ee_vel', 'osc_goal_pos', 'osc_goal_rot',
                                             'osc_gripper', 'osc_gains', 'osc_q0')}
    dd['osc_action'].copy_(torch.from_numpy(acts[1]))
    dd.osc(native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    assert not _np(dd['osc_error']).any()
    ranges = m.arrays['actuator_ctrlrange'][m.arrays['osc_actuator']].reshape(-1)
    worst = 0.0
    for w in range(nworld):
        inp = dict(mass=inputs['osc_mass'][w], jac=inputs['osc_jac'][w], q=inputs['osc_q'][w],
                   qvel=inputs['osc_qvel'][w], bias=inputs['osc_bias'][w], ee_pos=inputs['osc_ee_pos'][w],
                   ee_rot=inputs['osc_ee_rot'][w], ee_vel=inputs['osc_ee_vel'][w])
        err, tau, ctrl, rank, gp, gr, gg = O.osc(inp, acts[1][w], inputs['osc_gains'][w], inputs['osc_q0'][w], ranges,
                                                 inputs['osc_goal_pos'][w], inputs['osc_goal_rot'][w],
                                                 inputs['osc_gripper'][w], policy=True)
        assert err == 0
        worst = max(worst, rel_err(_np(dd['osc_tau'])[w], tau))
        assert np.allclose(_np(dd['osc_goal_pos'])[w], gp, rtol=0, atol=1e-12)
        assert np.allclose(_np(dd['osc_goal_rot'])[w], gr, rtol=0, atol=1e-12)
        assert np.array_equal(_np(dd['osc_rank'])[w], rank)
        np.testing.assert_allclose(_np(dd['ctrl'])[w, m.arrays['osc_actuator']], ctrl, rtol=1e-6, atol=1e-6)
    print(config, 'standalone osc tau rel', worst)
    assert worst < 1e-9


def test_osc_action_ranges_and_zero_rotation(gpu_available):
    """Configured action ranges (robosuite scale_action), different in every world, and actions
    whose rotation part is zero in half of the worlds: the in-kernel controller's policy substep
    against the oracle's FP64 OSC on the inputs the substep published, from the goal and gripper it
    started with: goal position and orientation within 1e-12, the zero-rotation worlds' orientation
    goal unchanged bit for bit, gripper exact, tau within 1e-9 relative."""
    import torch
    from libero_hip import scene as S, native
    from oracle import oracle as O
    nworld = 32
    sc = S.make_scene('c2', nworld, seed=2)
    sc.osc = dict(sc.osc, input_min=-2.0, input_max=2.0, output_min=[-0.1] * 3 + [-0.8] * 3,
                  output_max=[0.08] * 3 + [0.6] * 3)
    m, dd, od = _pair('c2', nworld, seed=2, scene=sc)
    assert m.osc_action_scaled == 1
    rng = np.random.default_rng(21)
    lo = rng.uniform(-2.0, 0.0, (nworld, 6))
    ranges = np.concatenate([lo, lo + rng.uniform(0.5, 3.0, (nworld, 6)), rng.uniform(-0.3, 0.0, (nworld, 6)),
                             rng.uniform(0.0, 0.4, (nworld, 6))], axis=1)
    # even worlds: rotation ranges centred on zero, so that a zero action is a zero rotation delta
    ranges[::2, 9:12] = np.abs(ranges[::2, 9:12]) + 0.5
    ranges[::2, 3:6] = -ranges[::2, 9:12]
    ranges[::2, 15:18] = -ranges[::2, 21:24]
    assert (ranges[:, :6] < ranges[:, 6:12]).all() and (ranges[:, 12:18] < ranges[:, 18:]).all()
    dd['osc_action_scale'].copy_(torch.from_numpy(ranges))
    acts = rng.uniform(-2.5, 2.5, (nworld, 7))
    acts[::2, 3:6] = 0.0
    before = {k: _np(dd[k]).copy() for k in ('osc_goal_pos', 'osc_goal_rot', 'osc_gripper')}
    # a goal orientation away from the current pose, so that keeping it is visible
    from scipy.spatial.transform import Rotation
    turn = np.stack([(Rotation.from_rotvec(rng.normal(size=3) * 0.2).as_matrix()
                      @ before['osc_goal_rot'][w].reshape(3, 3)).reshape(-1) for w in range(nworld)])
    dd['osc_goal_rot'].copy_(torch.from_numpy(turn))
    before['osc_goal_rot'] = turn
    dd['osc_action'].copy_(torch.from_numpy(acts))
    dd.control_step(1, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    assert not _np(dd['osc_error']).any()
    crange = m.arrays['actuator_ctrlrange'][m.arrays['osc_actuator']].reshape(-1)
    worst = 0.0
    for w in range(nworld):
        inp = {k: _np(dd['osc_' + k])[w] for k in ('mass', 'jac', 'q', 'qvel', 'bias', 'ee_pos', 'ee_rot', 'ee_vel')}
        err, tau, ctrl, rank, gp, gr, gg = O.osc(inp, acts[w], _np(dd['osc_gains'])[w], _np(dd['osc_q0'])[w], crange,
                                                 before['osc_goal_pos'][w], before['osc_goal_rot'][w],
                                                 before['osc_gripper'][w], policy=True,
                                                 speed=float(np.float32(m.osc_gripper_speed)),   # a model float
                                                 action_scale=ranges[w])
        assert err == 0
        np.testing.assert_allclose(_np(dd['osc_goal_pos'])[w], gp, rtol=0, atol=1e-12)
        np.testing.assert_allclose(_np(dd['osc_goal_rot'])[w], gr, rtol=0, atol=1e-12)
        if w % 2 == 0:
            np.testing.assert_array_equal(_np(dd['osc_goal_rot'])[w], turn[w])
        else:
            assert np.abs(_np(dd['osc_goal_rot'])[w] - turn[w]).max() > 1e-3
        np.testing.assert_array_equal(_np(dd['osc_gripper'])[w], gg)
        worst = max(worst, rel_err(_np(dd['osc_tau'])[w], tau))
    print('configured ranges: osc tau rel', worst)
    assert worst < 1e-9
