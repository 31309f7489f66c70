"""Write tests/golden/osc_fixture.npz: FP64 OSC golden vectors from numpy alone (and
osc_fixture_ndof.npz for other joint counts, osc_policy_fixture.npz for policy steps).

Inputs follow the reference's fixture recipe (tests/cuda/osc_reference_fixture.py:36-66 of the
reference: seed 327, 4 cases x 2 worlds x 3 transitions, SPD masses, rank-deficient / tiny / zero
Jacobians, a 0.07 rad goal rotation).  Expected outputs use robosuite's published formulas
(opspace_matrices, nullspace_torques, orientation_error; restated in the reference fixture at
:9-33) with numpy.linalg.inv / numpy.linalg.pinv, which is what the reference compares against.
robosuite itself is not installed here; the formulas are restated below.

Run: python tests/golden/make_osc_fixture.py
"""
import math
from pathlib import Path

import numpy as np

# robosuite's OSC_POSE defaults (controllers/config/osc_pose.json): input_min, input_max,
# output_min, output_max of the 6-D pose delta
DEFAULT_RANGES = np.r_[np.full(6, -1.0), np.full(6, 1.0), [-0.05] * 3 + [-0.5] * 3, [0.05] * 3 + [0.5] * 3]


def orientation_error(desired, current):
    rc = [current[:, k] for k in range(3)]
    rd = [desired[:, k] for k in range(3)]
    return 0.5 * (np.cross(rc[0], rd[0]) + np.cross(rc[1], rd[1]) + np.cross(rc[2], rd[2]))


def opspace_matrices(m, jf, jp, jr):
    mi = np.linalg.inv(m)
    lf = np.linalg.pinv(jf @ mi @ jf.T)
    lp = np.linalg.pinv(jp @ mi @ jp.T)
    lr = np.linalg.pinv(jr @ mi @ jr.T)
    jbar = mi @ jf.T @ lf
    return lf, lp, lr, np.eye(jf.shape[1]) - jbar @ jf


def nullspace_torques(m, n, q0, q, qd, kp=10.0):
    kv = 2 * np.sqrt(kp)
    return n.T @ (m @ (kp * (q0 - q) - kv * qd))


def expected(v, w, n=7):
    m, j = v['pm'][w].reshape(n, n), v['pj'][w].reshape(6, n)
    lf, lp, lr, n = opspace_matrices(m, j, j[:3], j[3:])
    pos = v['goal_pos'][w] - v['pp'][w]
    ori = orientation_error(v['goal_rot'][w].reshape(3, 3), v['pr'][w].reshape(3, 3))
    desired = v['gains'][w, :6] * np.r_[pos, ori] - v['gains'][w, 6:] * v['pe'][w]
    nt = nullspace_torques(m, n, v['q0'][w], v['pq'][w], v['pv'][w])
    tau = j.T @ np.r_[lp @ desired[:3], lr @ desired[3:]] + v['bias'][w] + nt
    a = j @ np.linalg.inv(m) @ j.T
    ranks = [int(np.sum((s := np.linalg.svd(x, compute_uv=False)) > 1e-15 * s.max())) if np.any(x) else 0
             for x in (a, a[:3, :3], a[3:, 3:])]
    return tau, lf, lp, lr, n, ranks


def scale_action(action, ranges):
    """robosuite Controller.scale_action (controllers/base_controller.py)."""
    in_min, in_max, out_min, out_max = np.asarray(ranges, float).reshape(4, 6)
    scale = abs(out_max - out_min) / abs(in_max - in_min)
    out_transform = (out_max + out_min) / 2.0
    in_transform = (in_max + in_min) / 2.0
    action = np.clip(action, in_min, in_max)
    return (action - in_transform) * scale + out_transform


def axisangle2quat(vec):
    """robosuite transform_utils.axisangle2quat: (x, y, z, w), identity for a zero vector."""
    angle = np.linalg.norm(vec)
    if math.isclose(angle, 0.0):
        return np.array([0.0, 0.0, 0.0, 1.0])
    axis = vec / angle
    q = np.zeros(4)
    q[3] = np.cos(angle / 2.0)
    q[:3] = axis * np.sin(angle / 2.0)
    return q


def quat2mat(quaternion):
    """robosuite transform_utils.quat2mat, which works in float32, with the scalar promotion of the
    numpy 1.x it ran on: `1.0 - q2[i, i] - ...` of a Python float and float32 scalars is float64
    (numpy 2 keeps float32 there, so the float64 steps are written out)."""
    q = np.asarray(quaternion).copy().astype(np.float32)[[3, 0, 1, 2]]
    n = np.dot(q, q)
    if n < np.finfo(float).eps * 4.0:
        return np.identity(3)
    q *= np.float32(math.sqrt(2.0 / float(n)))
    q2 = np.outer(q, q)
    d = lambda i, j: (1.0 - float(q2[i, i])) - float(q2[j, j])  # noqa: E731
    return np.array([[d(2, 3), q2[1, 2] - q2[3, 0], q2[1, 3] + q2[2, 0]],
                     [q2[1, 2] + q2[3, 0], d(1, 3), q2[2, 3] - q2[1, 0]],
                     [q2[1, 3] - q2[2, 0], q2[2, 3] + q2[1, 0], d(1, 2)]], dtype=np.float64)


def set_goal(action, ranges, ee_pos, ee_rot, goal_pos, goal_rot):
    """robosuite OSC.set_goal with delta actions: goal_pos = ee_pos + delta[:3]
    (set_goal_position); the goal orientation moves to quat2mat(axisangle2quat(delta[3:])) ee_rot
    (set_goal_orientation) only if some rotation component is not isclose to 0, else is kept."""
    delta = scale_action(np.asarray(action, float)[:6], ranges)
    new_pos = np.asarray(ee_pos, float) + delta[:3]
    if sum(0.0 if math.isclose(e, 0.0) else 1.0 for e in delta[3:]) > 0.0:
        new_rot = np.dot(quat2mat(axisangle2quat(delta[3:])), np.asarray(ee_rot, float).reshape(3, 3))
    else:
        new_rot = np.asarray(goal_rot, float).reshape(3, 3).copy()
    return new_pos, new_rot.reshape(-1)


def gripper_step(state, a6, speed, ctrlrange):
    """robosuite PandaGripper.format_action (state += [-1, 1] speed sign(a), clipped to [-1, 1]) and
    the robot's mapping of the state onto the actuators' control range (bias + weight state)."""
    state = np.clip(np.asarray(state, float) + np.array([-1.0, 1.0]) * speed * np.sign(a6), -1.0, 1.0)
    lo, hi = np.asarray(ctrlrange, float).reshape(2, 2).T
    return state, 0.5 * (hi + lo) + 0.5 * (hi - lo) * state


def main_policy(path):
    """Policy steps (osc_policy_fixture.npz): 7-joint inputs as the recipe above, actions partly
    outside the input range, some with a zero rotation part, robosuite's default ranges and
    random asymmetric ones; expected goal, gripper state, tau and ctrl."""
    rng = np.random.default_rng(329)
    keys = ('pm', 'pj', 'pq', 'pv', 'bias', 'q0', 'pp', 'pr', 'pe', 'goal_pos0', 'goal_rot0', 'grip0', 'action',
            'ranges', 'scaled', 'speed', 'gains', 'range', 'goal_pos', 'goal_rot', 'grip', 'tau', 'ctrl')
    out = {k: [] for k in keys}
    from scipy.spatial.transform import Rotation
    for case in range(24):
        m = rng.normal(size=(7, 7))
        m = m @ m.T + np.eye(7) * 2
        j = rng.normal(size=(6, 7))
        ee_rot = Rotation.from_rotvec(rng.normal(size=3)).as_matrix().reshape(-1)
        goal_rot0 = Rotation.from_rotvec(rng.normal(size=3) * 0.2).as_matrix() @ ee_rot.reshape(3, 3)
        action = rng.uniform(-1.6, 1.6, size=7)
        if case % 4 == 1:
            action[3:6] = 0.0                       # no rotation: the goal orientation is kept
        if case % 4 == 2:
            action[6] = 0.0                         # no gripper motion
        scaled = case >= 12
        ranges = DEFAULT_RANGES.copy()
        if scaled:
            lo = rng.uniform(-2.0, 0.0, 6)
            ranges = np.r_[lo, lo + rng.uniform(0.5, 3.0, 6), rng.uniform(-0.3, 0.0, 6), rng.uniform(0.0, 0.4, 6)]
        speed = 0.01 if case % 3 else 0.05
        crange = np.r_[np.tile([-87.0, 87.0], 7), [0.0, 0.04, -0.04, 0.0]]
        v = dict(pm=m, pj=j, pq=rng.normal(size=7) * .1, pv=rng.normal(size=7) * .05, bias=rng.normal(size=7),
                 q0=rng.normal(size=7) * .1, pp=rng.normal(size=3) * .05, pr=ee_rot, pe=rng.normal(size=6) * .02,
                 goal_pos0=rng.normal(size=3) * .05, goal_rot0=goal_rot0.reshape(-1), grip0=rng.uniform(-1, 1, 2),
                 gains=np.r_[np.full(6, 150.), np.full(6, 2 * np.sqrt(150.))], range=crange)
        gp, gr = set_goal(action, ranges, v['pp'], v['pr'], v['goal_pos0'], v['goal_rot0'])
        tau = expected(dict((k, x[None]) for k, x in dict(v, goal_pos=gp, goal_rot=gr).items()), 0)[0]
        grip, gctrl = gripper_step(v['grip0'], action[6], speed, crange[14:18])
        v.update(action=action, ranges=ranges, scaled=np.int32(scaled), speed=np.float64(speed), goal_pos=gp,
                 goal_rot=gr, grip=grip, tau=tau, ctrl=np.r_[np.clip(tau, -87, 87), gctrl])
        for k in keys:
            out[k].append(np.asarray(v[k]).reshape(-1) if np.ndim(v[k]) else v[k])
    np.savez(path, **{k: np.array(x) for k, x in out.items()})
    print('wrote', path, len(out['tau']), 'cases')


def main(path):
    rng = np.random.default_rng(327)
    out = {k: [] for k in ('pm', 'pj', 'pq', 'pv', 'bias', 'q0', 'pp', 'pr', 'pe', 'goal_pos', 'goal_rot',
                           'gains', 'range', 'tau', 'lambda_full', 'lambda_pos', 'lambda_ori', 'nullspace', 'ranks')}
    for case in range(4):
        m = rng.normal(size=(2, 7, 7))
        m = m @ m.transpose(0, 2, 1) + np.eye(7) * 2
        j = rng.normal(size=(2, 6, 7))
        if case == 1:
            j[0, 4:] = 0
            j[1, 5:] = 0
        elif case == 2:
            j *= 1e-3
        elif case == 3:
            j[:] = 0
        rot = np.tile(np.eye(3).reshape(1, 9), (2, 1))
        c, s = np.cos(.07), np.sin(.07)
        goals = np.tile(np.array([[c, -s, 0], [s, c, 0], [0, 0, 1]]).reshape(1, 9), (2, 1))
        v = dict(pm=m.reshape(2, 49), pj=j.reshape(2, 42), pq=rng.normal(size=(2, 7)) * .1,
                 pv=rng.normal(size=(2, 7)) * .05, bias=rng.normal(size=(2, 7)),
                 q0=np.zeros((2, 7)), pp=rng.normal(size=(2, 3)) * .05, pr=rot,
                 pe=rng.normal(size=(2, 6)) * .02, goal_pos=rng.normal(size=(2, 3)) * .05,
                 goal_rot=goals, gains=np.tile(np.r_[np.full(6, 150.), np.full(6, 2 * np.sqrt(150.))], (2, 1)),
                 range=np.tile(np.array([-87., 87.]), (2, 9)))
        for step in range(3):
            if step == 2:
                v['pm'][1, 0] += .125        # the reference's third transition (non-symmetric input)
            for w in range(2):
                tau, lf, lp, lr, n, ranks = expected(v, w)
                for k in ('pm', 'pj', 'pq', 'pv', 'bias', 'q0', 'pp', 'pr', 'pe', 'goal_pos', 'goal_rot', 'gains', 'range'):
                    out[k].append(np.array(v[k][w], float))
                out['tau'].append(tau)
                out['lambda_full'].append(lf.reshape(-1))
                out['lambda_pos'].append(lp.reshape(-1))
                out['lambda_ori'].append(lr.reshape(-1))
                out['nullspace'].append(n.reshape(-1))
                out['ranks'].append(np.array(ranks, np.int32))
    np.savez(path, **{k: np.array(v) for k, v in out.items()})
    print('wrote', path, len(out['tau']), 'cases')


def main_ndof(path, dofs=(6, 8)):
    """The same recipe for arms of other joint counts (osc_fixture_ndof.npz): per case the joint
    count n, inputs padded to 8 joints (mass 8 x 8, Jacobian 6 x 8, n-vectors 8)."""
    rng = np.random.default_rng(328)
    keys = ('ndof', 'pm', 'pj', 'pq', 'pv', 'bias', 'q0', 'pp', 'pr', 'pe', 'goal_pos', 'goal_rot', 'gains',
            'range', 'tau', 'ranks')
    out = {k: [] for k in keys}
    pad = lambda x, size: np.r_[np.asarray(x, float).reshape(-1), np.zeros(size - np.asarray(x).size)]  # noqa: E731
    for n in dofs:
        for case in range(3):
            m = rng.normal(size=(2, n, n))
            m = m @ m.transpose(0, 2, 1) + np.eye(n) * 2
            j = rng.normal(size=(2, 6, n))
            if case == 1:
                j[0, 4:] = 0
                j[1, :, n - 1] = 0
            elif case == 2:
                j *= 1e-3
            c, s = np.cos(.05), np.sin(.05)
            v = dict(pm=m.reshape(2, n * n), pj=j.reshape(2, 6 * n), pq=rng.normal(size=(2, n)) * .1,
                     pv=rng.normal(size=(2, n)) * .05, bias=rng.normal(size=(2, n)), q0=rng.normal(size=(2, n)) * .1,
                     pp=rng.normal(size=(2, 3)) * .05, pr=np.tile(np.eye(3).reshape(1, 9), (2, 1)),
                     pe=rng.normal(size=(2, 6)) * .02, goal_pos=rng.normal(size=(2, 3)) * .05,
                     goal_rot=np.tile(np.array([[1, 0, 0], [0, c, -s], [0, s, c]]).reshape(1, 9), (2, 1)),
                     gains=np.tile(np.r_[np.full(6, 150.), np.full(6, 2 * np.sqrt(150.))], (2, 1)),
                     range=np.tile(np.array([-87., 87.]), (2, n + 2)))
            for w in range(2):
                tau, lf, lp, lr, nul, ranks = expected(v, w, n)
                out['ndof'].append(np.int32(n))
                for k, size in (('pm', 64), ('pj', 48), ('pq', 8), ('pv', 8), ('bias', 8), ('q0', 8), ('range', 20)):
                    out[k].append(pad(v[k][w], size))
                for k in ('pp', 'pr', 'pe', 'goal_pos', 'goal_rot', 'gains'):
                    out[k].append(np.array(v[k][w], float))
                out['tau'].append(pad(tau, 8))
                out['ranks'].append(np.array(ranks, np.int32))
    np.savez(path, **{k: np.array(v) for k, v in out.items()})
    print('wrote', path, len(out['tau']), 'cases')


if __name__ == '__main__':
    main(Path(__file__).resolve().parent / 'osc_fixture.npz')
    main_ndof(Path(__file__).resolve().parent / 'osc_fixture_ndof.npz')
    main_policy(Path(__file__).resolve().parent / 'osc_policy_fixture.npz')
