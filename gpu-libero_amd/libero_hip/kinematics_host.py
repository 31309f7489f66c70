"""Host (numpy, FP64) forward kinematics and mass matrix for model compilation.

Used once per model to derive the compile-time constants MuJoCo's ``mj_setConst`` produces
(``body_invweight0``, ``dof_invweight0``).  It follows MuJoCo's ``mj_kinematics``, ``mj_comPos``
and ``mj_crb`` in meaning (the reference's fused leaf for the same stages is
``gpu/cuda/fp32/fused_kinematic_mass.cu:110-447``).  It is not on the stepping path.
"""
from __future__ import annotations

import math
import numpy as np

from . import scene as S


def _quat2mat(q):
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _qmul(a, b):
    return np.array(S._qmul(a, b))


def forward_host(model, qpos):
    a = model.arrays
    nb, nv = model.nbody, model.nv
    xpos = np.zeros((nb, 3))
    xquat = np.zeros((nb, 4))
    xquat[0] = (1, 0, 0, 0)
    xmat = np.zeros((nb, 3, 3))
    xmat[0] = np.eye(3)
    xanchor = np.zeros((model.njnt, 3))
    xaxis = np.zeros((model.njnt, 3))
    for b in range(1, nb):
        p = a['body_parent'][b]
        pos = xpos[p] + xmat[p] @ a['body_pos'][b]
        quat = _qmul(xquat[p], a['body_quat'][b])
        for j in range(a['body_jntadr'][b], a['body_jntadr'][b] + a['body_jntnum'][b]):
            qa = a['jnt_qposadr'][j]
            t = a['jnt_type'][j]
            if t == S.FREE:
                pos = qpos[qa:qa + 3].copy()
                quat = qpos[qa + 3:qa + 7] / np.linalg.norm(qpos[qa + 3:qa + 7])
                xanchor[j] = pos
                xaxis[j] = (0, 0, 1)
                continue
            R = _quat2mat(quat)
            xanchor[j] = R @ a['jnt_pos'][j] + pos
            xaxis[j] = R @ a['jnt_axis'][j]
            if t == S.SLIDE:
                pos = pos + xaxis[j] * (qpos[qa] - a['qpos0'][qa])
            elif t == S.HINGE:
                ang = qpos[qa] - a['qpos0'][qa]
                ax = a['jnt_axis'][j]
                ql = np.array([math.cos(ang / 2), *(ax * math.sin(ang / 2))])
                quat = _qmul(quat, ql)
                pos = xanchor[j] - _quat2mat(quat) @ a['jnt_pos'][j]
        quat = quat / np.linalg.norm(quat)
        xpos[b], xquat[b], xmat[b] = pos, quat, _quat2mat(quat)
    xipos = np.array([xpos[b] + xmat[b] @ a['body_ipos'][b] for b in range(nb)])
    ximat = np.array([xmat[b] @ _quat2mat(a['body_iquat'][b]) for b in range(nb)])
    mass = a['body_mass']
    # subtree centres of mass
    msum = mass.copy()
    mcom = mass[:, None] * xipos
    for b in range(nb - 1, 0, -1):
        p = a['body_parent'][b]
        msum[p] += msum[b]
        mcom[p] += mcom[b]
    subtree_com = np.where(msum[:, None] > 1e-15, mcom / np.maximum(msum, 1e-15)[:, None], xipos)
    root = a['body_rootid']
    # motion subspaces (cdof) about the subtree com of the tree root, [angular; linear]
    cdof = np.zeros((nv, 6))
    for j in range(model.njnt):
        b = a['jnt_body'][j]
        d = a['jnt_dofadr'][j]
        off = subtree_com[root[b]] - xanchor[j]
        t = a['jnt_type'][j]
        if t == S.FREE:
            for k in range(3):
                cdof[d + k, 3 + k] = 1.0
            for k in range(3):
                ax = xmat[b][:, k]
                cdof[d + 3 + k] = np.r_[ax, np.cross(ax, off)]
        elif t == S.HINGE:
            cdof[d] = np.r_[xaxis[j], np.cross(xaxis[j], off)]
        elif t == S.SLIDE:
            cdof[d] = np.r_[0, 0, 0, xaxis[j]]
    # mass matrix as sum over bodies of J_b^T I_b J_b (brute force; compile time only)
    M = np.zeros((nv, nv))

    def jac(body, point):
        jacp = np.zeros((3, nv))
        jacr = np.zeros((3, nv))
        d = a['body_lastdof'][body]
        off = point - subtree_com[root[body]]
        while d >= 0:
            jacr[:, d] = cdof[d, :3]
            jacp[:, d] = cdof[d, 3:] + np.cross(cdof[d, :3], off)
            d = a['dof_parent'][d]
        return jacp, jacr

    for b in range(1, nb):
        jp, jr = jac(b, xipos[b])
        I = ximat[b] @ np.diag(a['body_inertia'][b]) @ ximat[b].T
        M += mass[b] * jp.T @ jp + jr.T @ I @ jr
    M += np.diag(a['dof_armature'])
    return dict(xpos=xpos, xquat=xquat, xmat=xmat, xipos=xipos, ximat=ximat,
                subtree_com=subtree_com, cdof=cdof, M_dense=M, jac=jac)
