"""Heterogeneous batches (per-world object counts): the oracle's masking of parked objects.

A world of a heterogeneous batch holds the same model as every other world, with the object slots
it does not use marked inactive in ``body_active`` and parked far below the floor.  Two facts pin
the oracle's treatment of them without restating its code:

* no contact ever involves an inactive body (its collision pairs are skipped);
* an inactive object is a free body under gravity alone, so semi-implicit Euler gives the closed
  form v_n = g dt n and z_n = z_0 + g dt^2 n (n + 1) / 2, with x, y and the orientation unchanged.
"""
import numpy as np

from helpers import make_oracle
from libero_hip import scene as S
from libero_hip.model import Model

O_FLAGS = 8 | 2   # bootstrap the controller goal, no control update


def test_parked_objects_never_collide_and_fall_freely():
    nworld = 8
    sc = S.make_scene('c5', nworld, seed=3)
    m = Model(sc)
    act = m.body_active
    assert act is not None and (act == 0).any() and (act == 1).sum(1).min() > 0
    nobj = (m.nq - 9) // 7
    first = m.nbody - nobj
    om, od = make_oracle(m, nworld)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, O_FLAGS)
    body = m.arrays['geom_body']
    dt, g = sc.options.timestep, sc.options.gravity[2]
    n = 0
    for _ in range(3):
        od.control_step(25, 2)
        n += 25
        for w in range(nworld):
            c = int(od['ncon'][w, 0])
            geoms = od['contact_geom'][w, :2 * c]
            assert act[w, body[geoms]].all(), 'contact with a parked body in world %d' % w
        for w in range(nworld):
            for k in range(nobj):
                if act[w, first + k]:
                    continue
                q = od['qpos'][w, 9 + 7 * k:16 + 7 * k]
                v = od['qvel'][w, 9 + 6 * k:15 + 6 * k]
                q0 = sc.init_qpos[w, 9 + 7 * k:16 + 7 * k]
                np.testing.assert_allclose(q[:2], q0[:2], rtol=0, atol=1e-12)
                np.testing.assert_allclose(q[2], q0[2] + g * dt * dt * n * (n + 1) / 2, rtol=1e-12)
                np.testing.assert_allclose(q[3:], q0[3:], rtol=0, atol=1e-12)
                np.testing.assert_allclose(v, [0, 0, g * dt * n, 0, 0, 0], rtol=1e-12, atol=1e-12)
    # the active objects did collide: the masking does not switch contacts off altogether
    assert od['ncon'][:, 0].sum() > 0
