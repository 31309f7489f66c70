"""Test helpers: paired GPU / oracle batches started from the same state."""
import numpy as np

from libero_hip import scene as S
from libero_hip.model import Model
from oracle import oracle as O


def rel_err(a, b, floor=1e-6):
    """Max-abs difference over max-abs reference (per row when 2-D), floored."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.ndim == 1:
        return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), floor))
    num = np.max(np.abs(a - b), axis=1)
    den = np.maximum(np.max(np.abs(b), axis=1), floor)
    return float(np.max(num / den))


def seeded_state(model, nworld, seed, qvel_scale=0.5):
    """Initial qpos from the scene plus seeded joint velocities (objects at rest)."""
    rng = np.random.default_rng(seed)
    sc = model.scene
    qpos = sc.init_qpos[:nworld].copy()
    qvel = np.zeros((nworld, model.nv))
    nr = model.osc_ndof + 2                  # the robot's dofs: arm joints and two fingers
    qvel[:, :nr] = rng.uniform(-qvel_scale, qvel_scale, size=(nworld, nr))
    return qpos, qvel


def make_oracle(model, nworld, fp32_model=False):
    om = O.OracleModel(model, fp32_model=fp32_model)
    od = O.OracleData(om, nworld)
    sc = model.scene
    od['osc_gains'][:] = np.r_[sc.osc['kp'], sc.osc['kd']]
    od['osc_q0'][:] = sc.osc['q0']
    od['body_active'][:] = 1 if model.body_active is None else model.body_active
    return om, od
