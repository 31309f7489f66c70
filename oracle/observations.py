"""CPU FP64 restatement of the device observation sampler -- TEST INFRASTRUCTURE ONLY.

Only tests/ import this module.  It restates, in numpy double precision, the reference's sampling of
an ordered observable plan (gpu/cuda/fp32/fused_observations.cu:39-168 pack_and_sample, the
ParallelClock path: clocks per spec, then the sampled specs in plan order) with robosuite's own
formulas for the pose operations (robosuite.utils.transform_utils quat2mat, mat2quat by the
dominant eigenvector of Bar-Itzhack's K via numpy.linalg.eigh, pose_inv, pose_in_A_to_pose_in_B,
mat2pose), which the device code computes in FP32 by other means (Shepperd's closed form).  The
clocks are FP32 as the reference's (elapsed, dt and period are float32 there): a sampling decision
is discrete, so it must round as the device's does.
"""
from __future__ import annotations

import numpy as np

EPS = np.finfo(float).eps * 4.0


def quat2mat(q):
    """robosuite quat2mat of an (x, y, z, w) quaternion."""
    q = np.asarray(q, float)[[3, 0, 1, 2]]
    n = np.dot(q, q)
    if n < EPS:
        return np.identity(3)
    q = q * np.sqrt(2.0 / n)
    q2 = np.outer(q, q)
    return np.array([[1.0 - q2[2, 2] - q2[3, 3], q2[1, 2] - q2[3, 0], q2[1, 3] + q2[2, 0]],
                     [q2[1, 2] + q2[3, 0], 1.0 - q2[1, 1] - q2[3, 3], q2[2, 3] - q2[1, 0]],
                     [q2[1, 3] - q2[2, 0], q2[2, 3] + q2[1, 0], 1.0 - q2[1, 1] - q2[2, 2]]])


def mat2quat(m):
    """robosuite mat2quat: (x, y, z, w), w >= 0, the eigenvector of the largest eigenvalue of K."""
    M = np.asarray(m, float)[:3, :3]
    m00, m01, m02 = M[0]
    m10, m11, m12 = M[1]
    m20, m21, m22 = M[2]
    K = np.array([[m00 - m11 - m22, 0.0, 0.0, 0.0],
                  [m01 + m10, m11 - m00 - m22, 0.0, 0.0],
                  [m02 + m20, m12 + m21, m22 - m00 - m11, 0.0],
                  [m21 - m12, m02 - m20, m10 - m01, m00 + m11 + m22]]) / 3.0
    w, V = np.linalg.eigh(K)
    q = V[[3, 0, 1, 2], np.argmax(w)]
    if q[0] < 0.0:
        q = -q
    return q[[1, 2, 3, 0]]


def pose_inv(pos, quat):
    """4x4 inverse of the pose (pos, quat x y z w)."""
    R = quat2mat(quat)
    T = np.identity(4)
    T[:3, :3] = R.T
    T[:3, 3] = -R.T @ np.asarray(pos, float)
    return T


def relative_pose(pos, quat, frame):
    """(position, quaternion) of the pose (pos, quat) expressed in the 4x4 frame `frame`."""
    P = np.identity(4)
    P[:3, :3] = quat2mat(quat)
    P[:3, 3] = pos
    Q = np.asarray(frame, float) @ P
    return Q[:3, 3], mat2quat(Q[:3, :3])


class Sampler:
    """Per-world observation state of a plan (libero_hip.observations.ObservationPlan)."""

    def __init__(self, plan, nworld):
        self.plan = plan
        self.offsets = plan.offsets
        self.ids = {s.name: i for i, s in enumerate(plan.specs)}
        ns, width = len(plan.specs), plan.width
        self.cache = np.zeros((nworld, width))
        self.observed = np.zeros((nworld, width))
        self.side = np.zeros((nworld, width))
        self.elapsed = np.zeros((nworld, ns), np.float32)
        self.sampled = np.zeros((nworld, ns), bool)
        self.present = np.zeros((nworld, ns), bool)
        self.events = np.zeros((nworld, ns), bool)

    def reset(self, worlds):
        for w in worlds:
            self.elapsed[w] = 0
            self.present[w] = False
            self.cache[w] = self.observed[w] = self.side[w] = 0

    def _source(self, spec, fields, w):
        qpos, qvel, site, xpos, xquat = (fields[k][w] for k in ('qpos', 'qvel', 'site_xpos', 'xpos', 'xquat'))
        op, i = spec.operation, spec.indices
        if op == 'qpos':
            return qpos[list(i)]
        if op == 'qvel':
            return qvel[list(i)]
        if op == 'site_pos':
            return site[3 * i[0]:3 * i[0] + 3]
        if op == 'body_pos':
            return xpos[3 * i[0]:3 * i[0] + 3]
        if op == 'body_quat':
            return xquat[4 * i[0]:4 * i[0] + 4][[1, 2, 3, 0]]
        raise NotImplementedError(op)

    def sample(self, fields, dt, worlds, force=False):
        """One sampling call: fields are the raw arrays (nworld, width) of qpos, qvel, site_xpos,
        xpos, xquat."""
        for w in worlds:
            take = []
            for s, spec in enumerate(self.plan.specs):
                self.events[w, s] = False
                t = False
                if spec.enabled:
                    period = np.float32(spec.period)
                    e = np.float32(self.elapsed[w, s] + np.float32(dt))
                    due = e >= period
                    t = (not self.sampled[w, s] and period >= e) or force or (due and not self.sampled[w, s])
                    self.elapsed[w, s] = np.fmod(e, period) if due else e
                    self.sampled[w, s] = False if due else (True if t else self.sampled[w, s])
                take.append(t)
            for s, spec in enumerate(self.plan.specs):
                if not take[s]:
                    continue
                at, n = self.offsets[spec.name], spec.width
                deps = [self.offsets[d] for d in spec.dependencies]
                here = all(self.present[w, self.ids[d]] for d in spec.dependencies)
                c = self.cache[w]
                value = np.zeros(n)
                if spec.operation in ('qpos', 'qvel', 'site_pos', 'body_pos', 'body_quat'):
                    value = self._source(spec, fields, w)
                elif spec.operation in ('cos', 'sin'):
                    if here:
                        f = np.cos if spec.operation == 'cos' else np.sin
                        value = f(c[deps[0]:deps[0] + n])
                elif spec.operation == 'inverse_pose':
                    value = (pose_inv(c[deps[0]:deps[0] + 3], c[deps[1]:deps[1] + 4]) if here else np.identity(4)).reshape(-1)
                elif spec.operation == 'relative_pos':
                    if here:
                        value, q = relative_pose(c[deps[0]:deps[0] + 3], c[deps[1]:deps[1] + 4],
                                                 c[deps[2]:deps[2] + 16].reshape(4, 4))
                        self.side[w, at:at + 4] = q
                elif spec.operation == 'relative_quat':
                    if here:
                        value = self.side[w, deps[0]:deps[0] + 4]
                c[at:at + n] = value
                self.observed[w, at:at + n] = value
                self.present[w, s] = self.events[w, s] = True
