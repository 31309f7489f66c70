"""Write tests/golden/osc_fixture.npz: FP64 OSC golden vectors from numpy alone.

Inputs follow the reference's fixture recipe (tests/cuda/osc_reference_fixture.py:36-66 of the
reference: seed 327, 4 cases x 2 worlds x 3 transitions, SPD masses, rank-deficient / tiny / zero
Jacobians, a 0.07 rad goal rotation).  Expected outputs use robosuite's published formulas
(opspace_matrices, nullspace_torques, orientation_error; restated in the reference fixture at
:9-33) with numpy.linalg.inv / numpy.linalg.pinv, which is what the reference compares against.
robosuite itself is not installed here; the formulas are restated below.

Run: python tests/golden/make_osc_fixture.py
"""
from pathlib import Path

import numpy as np


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
