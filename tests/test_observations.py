"""Observation plan, host packaging and the CPU restatement of the device sampler (no GPU).

* the default plan's order, widths and device metadata (gather sources and dependency offsets);
* pack_observations keeps plan order and concatenates each modality's active observables;
* the numpy sampler (oracle/observations.py), pinned independently of its own formulas:
  quaternion <-> matrix against scipy's Rotation, inverse pose times pose = identity, the
  end-effector's pose in its own frame = identity, and robosuite's clock law (a spec samples at the
  first call of each sampling period; forced calls always sample).
"""
import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from libero_hip import observations as OB, scene as S
from libero_hip.model import Model
from oracle import observations as OO


def test_default_plan_layout():
    m = Model(S.make_scene('c3', 2))
    plan = OB.default_plan(m)
    names = [s.name for s in plan.specs]
    assert names[:8] == ['robot0_joint_pos', 'robot0_joint_pos_cos', 'robot0_joint_pos_sin', 'robot0_joint_vel',
                         'robot0_eef_pos', 'robot0_eef_quat', 'robot0_gripper_qpos', 'robot0_gripper_qvel']
    assert names[8] == 'world_pose_in_gripper' and not plan.specs[8].active
    objects = [b.name for b in m.scene.bodies if b.joints and b.joints[0].type == S.FREE]
    assert len(objects) == 6 and names[9:13] == [objects[0] + '_pos', objects[0] + '_quat',
                                                  objects[0] + '_to_robot0_eef_pos', objects[0] + '_to_robot0_eef_quat']
    assert plan.width == 7 * 4 + 3 + 4 + 2 + 2 + 16 + 6 * 14
    assert all(abs(s.period - 0.05) < 1e-12 for s in plan.specs)     # 20 Hz control
    meta = OB.plan_metadata(plan, m)
    assert list(meta['op'][:9]) == [0, 1, 2, 0, 0, 0, 0, 0, 3]
    # eef quaternion: the hand body's xquat reordered to x y z w
    hand = int(m.arrays['site_body'][m.osc_site])
    k = meta['index_offset'][5]
    assert list(meta['indices'][k:k + 4]) == [(4 << 24) | (4 * hand + j) for j in (1, 2, 3, 0)]
    # cos reads the joint positions; relative_pos reads pos, quat and the inverse pose
    off = plan.offsets
    assert meta['dep0'][1] == off['robot0_joint_pos']
    assert (meta['dep0'][11], meta['dep1'][11], meta['dep2'][11]) == (off[objects[0] + '_pos'], off[objects[0] + '_quat'],
                                                                      off['world_pose_in_gripper'])
    assert list(meta['presence'][33:36]) == [9, 10, 8]


def test_plan_validation():
    spec = OB.ObservableSpec('a', 'x', 'cos', 2, dependencies=('b',))
    with pytest.raises(ValueError):
        OB.ObservationPlan((spec,)).validate()
    with pytest.raises(ValueError):
        OB.ObservationPlan((OB.ObservableSpec('a', 'x', 'qpos', 0),)).validate()
    m = Model(S.make_scene('c2', 2))
    bad = OB.ObservationPlan((OB.ObservableSpec('q', 'x', 'qpos', 1, (m.nq,)),)).validate()
    with pytest.raises(ValueError):
        OB.plan_metadata(bad, m)


def test_pack_observations_order_and_groups():
    m = Model(S.make_scene('c3', 2))
    plan = OB.default_plan(m)
    values = np.arange(plan.width, dtype=float)
    out = OB.pack_observations(plan, values)
    off = plan.offsets
    assert 'world_pose_in_gripper' not in out                         # inactive
    np.testing.assert_array_equal(out['robot0_eef_quat'], values[off['robot0_eef_quat']:off['robot0_eef_quat'] + 4])
    proprio = np.concatenate([out[s.name] for s in plan.specs if s.modality == 'robot0_proprio'])
    np.testing.assert_array_equal(out['robot0_proprio-state'], proprio)
    keys = [k for k in out if not k.endswith('-state')]
    assert keys == [s.name for s in plan.specs if s.active]


def test_quaternion_matrix_against_scipy():
    rng = np.random.default_rng(0)
    for _ in range(200):
        q = rng.normal(size=4)
        q /= np.linalg.norm(q)
        R = OO.quat2mat(q)
        np.testing.assert_allclose(R, Rotation.from_quat(q).as_matrix(), atol=1e-12)
        want = Rotation.from_matrix(R).as_quat()
        want = want if want[3] >= 0 else -want
        np.testing.assert_allclose(OO.mat2quat(R), want, atol=1e-9)


def test_pose_identities():
    rng = np.random.default_rng(1)
    for _ in range(50):
        q = rng.normal(size=4)
        q /= np.linalg.norm(q)
        p = rng.normal(size=3)
        T = np.identity(4)
        T[:3, :3] = Rotation.from_quat(q).as_matrix()
        T[:3, 3] = p
        np.testing.assert_allclose(OO.pose_inv(p, q) @ T, np.identity(4), atol=1e-12)
        pos, quat = OO.relative_pose(p, q, OO.pose_inv(p, q))
        np.testing.assert_allclose(pos, 0, atol=1e-12)
        np.testing.assert_allclose(np.abs(quat), [0, 0, 0, 1], atol=1e-9)


def test_clock_samples_at_the_start_of_each_period():
    """robosuite's Observable.update: a spec samples at its first update of every sampling period
    (period 25 calls here), and every forced call samples."""
    spec = OB.ObservableSpec('q', 'x', 'qpos', 1, (0,), period=0.05)
    plan = OB.ObservationPlan((spec,)).validate()
    smp = OO.Sampler(plan, 1)
    fields = dict(qpos=np.zeros((1, 1)), qvel=np.zeros((1, 1)), site_xpos=np.zeros((1, 3)), xpos=np.zeros((1, 3)),
                  xquat=np.zeros((1, 4)))
    hits = []
    for k in range(100):
        fields['qpos'][0, 0] = k
        smp.sample(fields, 0.002, [0])
        hits.append(bool(smp.events[0, 0]))
    assert [k for k, h in enumerate(hits) if h] == [0, 25, 50, 75]
    assert smp.observed[0, 0] == 75
    smp.sample(fields, 0.002, [0], force=True)
    assert smp.events[0, 0] and smp.observed[0, 0] == 99
