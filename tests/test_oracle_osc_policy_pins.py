"""Pins of the oracle's OSC policy step (goal update, action scaling, gripper) by robosuite's
documented semantics, with no code shared with the oracle.

The oracle restates the reference's controller (gpu/cuda/control/osc_solver.cu:38-47 action scaling,
:278-306 rotation_delta, :570-583 goal update, :667-673 gripper).  These tests check it against:

* scipy's rotation vectors: the goal orientation is R(delta) ee_rot with R the rotation by the
  vector delta (half the clipped action, default ranges): left multiplication, the full rotation
  vector as the axis-angle (not twice or half of it), within the float32 rounding of robosuite's
  quat2mat;
* a numpy restatement of robosuite 1.4's OSC.set_goal, scale_action, axisangle2quat, quat2mat and
  PandaGripper.format_action (tests/golden/make_osc_fixture.py), through the golden vectors it wrote
  and on random cases here;
* closed forms: goal_pos = ee_pos + 0.05 clip(a); a zero rotation part keeps the previous goal
  orientation (robosuite updates it only when some component is nonzero); NaN propagates; the
  gripper state walks by the speed and saturates at +-1, ctrl = mid + half state.
"""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / 'golden'


def _mk():
    spec = importlib.util.spec_from_file_location('mk_osc', GOLDEN / 'make_osc_fixture.py')
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    return mk


def _case(rng, n=7):
    m = rng.normal(size=(n, n))
    m = m @ m.T + 2 * np.eye(n)
    ee_rot = Rotation.from_rotvec(rng.normal(size=3)).as_matrix()
    inputs = dict(mass=m, jac=rng.normal(size=(6, n)), q=rng.normal(size=n) * .1, qvel=rng.normal(size=n) * .05,
                  bias=rng.normal(size=n), ee_pos=rng.normal(size=3) * .3, ee_rot=ee_rot, ee_vel=rng.normal(size=6) * .02)
    goal_rot0 = Rotation.from_rotvec(rng.normal(size=3) * .3).as_matrix() @ ee_rot
    return inputs, goal_rot0


GAINS = np.r_[np.full(6, 150.), np.full(6, 2 * np.sqrt(150.))]
CRANGE = np.r_[np.tile([-87., 87.], 7), [0.0, 0.04, -0.04, 0.0]]


def _policy(inputs, action, goal_rot0, gripper=(0.0, 0.0), **kw):
    err, tau, ctrl, rank, gp, gr, gg = O.osc(inputs, action, GAINS, np.zeros(7), CRANGE, np.zeros(3), goal_rot0,
                                             np.asarray(gripper, float), policy=True, **kw)
    assert err == 0
    return gp, gr.reshape(3, 3), gg, tau, ctrl


def test_goal_update_against_rotation_vectors():
    """Default ranges, actions partly outside [-1, 1]: goal_pos = ee + 0.05 clip(a[:3]) exactly as
    the FP64 sum, goal_rot = Rotation.from_rotvec(0.5 clip(a[3:6])) @ ee_rot within the float32
    rounding of robosuite's quat2mat (and orthonormal to that rounding)."""
    rng = np.random.default_rng(11)
    for _ in range(60):
        inputs, goal_rot0 = _case(rng)
        a = rng.uniform(-2.5, 2.5, size=7)
        gp, gr, *_ = _policy(inputs, a, goal_rot0)
        np.testing.assert_array_equal(gp, inputs['ee_pos'] + 0.05 * np.clip(a[:3], -1, 1))
        want = Rotation.from_rotvec(0.5 * np.clip(a[3:6], -1, 1)).as_matrix() @ inputs['ee_rot']
        assert np.abs(gr - want).max() < 1e-6
        assert np.abs(gr @ gr.T - np.eye(3)).max() < 1e-6


def test_goal_update_against_robosuite_restatement():
    """The same goal, to the last float32 rounding step, as the numpy restatement of robosuite's
    set_goal (float32 quat2mat), for default and random asymmetric ranges."""
    mk = _mk()
    rng = np.random.default_rng(12)
    for i in range(60):
        inputs, goal_rot0 = _case(rng)
        a = rng.uniform(-2.5, 2.5, size=7)
        ranges = mk.DEFAULT_RANGES.copy()
        if i % 2:
            lo = rng.uniform(-2.0, 0.0, 6)
            ranges = np.r_[lo, lo + rng.uniform(0.5, 3.0, 6), rng.uniform(-0.3, 0.0, 6), rng.uniform(0.0, 0.4, 6)]
        gp, gr, *_ = _policy(inputs, a, goal_rot0, action_scale=ranges)
        wp, wr = mk.set_goal(a, ranges, inputs['ee_pos'], inputs['ee_rot'], None, goal_rot0)
        np.testing.assert_allclose(gp, wp, rtol=0, atol=1e-15)
        assert np.abs(gr.reshape(-1) - wr).max() < 2e-7, i


def test_default_ranges_given_explicitly_are_bit_identical():
    """robosuite's default ranges passed as ranges give the same goal and torque bit for bit as the
    built-in defaults (the scaling formula reduces to 0.05 a and 0.5 a exactly)."""
    mk = _mk()
    rng = np.random.default_rng(13)
    for _ in range(20):
        inputs, goal_rot0 = _case(rng)
        a = rng.uniform(-2, 2, size=7)
        x = _policy(inputs, a, goal_rot0)
        y = _policy(inputs, a, goal_rot0, action_scale=mk.DEFAULT_RANGES)
        for u, v in zip(x, y):
            np.testing.assert_array_equal(u, v)


def test_zero_rotation_keeps_the_goal_orientation():
    """A rotation part of exact zeros leaves the previous goal orientation as it was (robosuite's
    set_goal); the position goal still moves.  One nonzero component rotates about that axis."""
    rng = np.random.default_rng(14)
    for _ in range(10):
        inputs, goal_rot0 = _case(rng)
        a = np.r_[rng.uniform(-1, 1, 3), 0.0, 0.0, 0.0, 0.5]
        gp, gr, *_ = _policy(inputs, a, goal_rot0)
        np.testing.assert_array_equal(gr, goal_rot0)
        np.testing.assert_array_equal(gp, inputs['ee_pos'] + 0.05 * a[:3])
        b = a.copy()
        b[4] = 0.6
        _, gr, *_ = _policy(inputs, b, goal_rot0)
        want = Rotation.from_rotvec([0.0, 0.3, 0.0]).as_matrix() @ inputs['ee_rot']
        assert np.abs(gr - want).max() < 1e-6
    # a range whose output centre is off zero maps a zero action to a nonzero rotation
    mk = _mk()
    inputs, goal_rot0 = _case(rng)
    ranges = mk.DEFAULT_RANGES.copy()
    ranges[18 + 5] = 0.7                       # output_max of the z rotation: centre 0.1
    _, gr, *_ = _policy(inputs, np.zeros(7), goal_rot0, action_scale=ranges)
    want = Rotation.from_rotvec([0.0, 0.0, 0.1]).as_matrix() @ inputs['ee_rot']
    assert np.abs(gr - want).max() < 1e-6


def test_nan_actions_propagate():
    """NaN survives clipping (as the reference's clip and numpy's): a NaN position component makes
    that goal coordinate NaN only; a NaN rotation component makes the goal orientation NaN."""
    rng = np.random.default_rng(15)
    inputs, goal_rot0 = _case(rng)
    a = np.r_[np.nan, 0.2, -0.3, 0.1, 0.2, 0.3, 1.0]
    gp, gr, *_ = _policy(inputs, a, goal_rot0)
    assert np.isnan(gp[0]) and np.isfinite(gp[1:]).all() and np.isfinite(gr).all()
    a = np.r_[0.1, 0.2, -0.3, 0.1, np.nan, 0.3, 1.0]
    gp, gr, *_ = _policy(inputs, a, goal_rot0)
    assert np.isfinite(gp).all() and np.isnan(gr).all()


def test_gripper_walks_by_speed_and_saturates():
    """Forty policy steps with positive, negative, zero and NaN gripper commands: the state moves by
    [-1, +1] speed sign(a6) per step, clipped to [-1, 1]; ctrl of the two gripper actuators is the
    centre of their range plus half its width times the state."""
    rng = np.random.default_rng(16)
    inputs, goal_rot0 = _case(rng)
    for speed in (0.01, 0.3):
        state = np.array([0.2, -0.4])
        cmds = [1.0] * 12 + [-0.5] * 15 + [0.0] * 3 + [2.0] * 10
        for a6 in cmds:
            a = np.r_[np.zeros(6), a6]
            *_, gg, tau, ctrl = _policy(inputs, a, goal_rot0, gripper=state, speed=speed)
            state = np.clip(state + np.array([-1.0, 1.0]) * speed * np.sign(a6), -1, 1)
            np.testing.assert_array_equal(gg, state)
            lo, hi = CRANGE[14::2], CRANGE[15::2]
            np.testing.assert_allclose(ctrl[7:], 0.5 * (hi + lo) + 0.5 * (hi - lo) * state, rtol=0, atol=1e-15)
        if speed > 0.1:
            assert np.abs(state).max() == 1.0        # the fast walk reached the clip
    *_, gg, _, ctrl = _policy(inputs, np.r_[np.zeros(6), np.nan], goal_rot0, gripper=(0.1, 0.1))
    assert np.isnan(gg).all() and np.isnan(ctrl[7:]).all()


def test_policy_golden_fixture():
    """Golden vectors of numpy alone (robosuite's set_goal, scale_action, quat2mat in float32,
    PandaGripper.format_action and the OSC torque): goal within float32 rounding, gripper exact,
    ctrl the clipped torques and gripper controls.  The torque of the policy step carries the goal's
    float32 rounding times the gains (within 1e-6 relative); from the fixture's own goal (the
    same controller without the policy update) it is within 1e-9."""
    f = np.load(GOLDEN / 'osc_policy_fixture.npz')
    assert len(f['tau']) == 24 and f['scaled'].sum() == 12
    assert (f['action'][:, 3:6] == 0).all(axis=1).sum() == 6
    for i in range(len(f['tau'])):
        inputs = dict(mass=f['pm'][i], jac=f['pj'][i], q=f['pq'][i], qvel=f['pv'][i], bias=f['bias'][i],
                      ee_pos=f['pp'][i], ee_rot=f['pr'][i], ee_vel=f['pe'][i])
        scale = f['ranges'][i] if f['scaled'][i] else None
        err, tau, ctrl, rank, gp, gr, gg = O.osc(inputs, f['action'][i], f['gains'][i], f['q0'][i], f['range'][i],
                                                 f['goal_pos0'][i], f['goal_rot0'][i], f['grip0'][i], policy=True,
                                                 speed=float(f['speed'][i]), action_scale=scale)
        assert err == 0, i
        np.testing.assert_allclose(gp, f['goal_pos'][i], rtol=0, atol=1e-15, err_msg='case %d' % i)
        assert np.abs(gr - f['goal_rot'][i]).max() < 2e-7, i
        np.testing.assert_array_equal(gg, f['grip'][i])
        ref = f['tau'][i]
        assert np.max(np.abs(tau - ref)) <= 1e-6 * np.max(np.abs(ref)), i
        np.testing.assert_allclose(ctrl[7:], f['ctrl'][i][7:], rtol=0, atol=1e-15)
        err, tau, ctrl, *_ = O.osc(inputs, f['action'][i], f['gains'][i], f['q0'][i], f['range'][i],
                                   f['goal_pos'][i], f['goal_rot'][i], f['grip'][i], policy=False)
        assert err == 0, i
        assert np.max(np.abs(tau - ref)) <= 1e-9 * np.max(np.abs(ref)), i
        np.testing.assert_allclose(ctrl[:7], f['ctrl'][i][:7], rtol=0, atol=1e-9 * np.max(np.abs(ref)))


def test_policy_fixture_generator_is_deterministic(tmp_path):
    mk = _mk()
    mk.main_policy(tmp_path / 'p.npz')
    new, old = np.load(tmp_path / 'p.npz'), np.load(GOLDEN / 'osc_policy_fixture.npz')
    for k in old.files:
        np.testing.assert_allclose(new[k], old[k], rtol=1e-12, atol=1e-14, err_msg=k)


def test_model_ranges_validation():
    """The model compiler packs robosuite's ranges as the reference's osc_action_config does and
    refuses non-finite ranges or input_min >= input_max with the reference's error."""
    from libero_hip.model import osc_action_ranges
    mk = _mk()
    scaled, r = osc_action_ranges({})
    assert scaled == 0
    np.testing.assert_array_equal(r, mk.DEFAULT_RANGES)
    scaled, r = osc_action_ranges({'input_min': -2.0, 'output_max': [0.1] * 6})
    assert scaled == 1 and (r[:6] == -2).all() and (r[18:] == 0.1).all() and (r[6:12] == 1).all()
    for bad in ({'input_min': 1.0}, {'input_max': [1, 1, 1, 1, 1, -1.5]}, {'output_min': np.nan}):
        with pytest.raises(ValueError, match='input_min < input_max'):
            osc_action_ranges(bad)
