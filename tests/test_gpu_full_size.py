"""The workspace route at the benchmark's full size (C3, N = 4096), through properties that do not
depend on the batch size.

The oracle is too slow to follow 4096 worlds, and the parity tests check the physics on small
batches; what changes with the batch size is the addressing (high world indices into the workspace
slabs, the shared image slab, a full grid of resident worlds).  So, at N = 4096:

* worlds given the same state and actions end one control step bit-identical wherever they sit in
  the batch (first, middle, last slab), and bit-identical to the same world run in a batch of 16;
* no overflow bit beyond the Newton / line-search iteration caps, every field finite;
* every world touches something (the homogeneous C3 batch rests objects on the table).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FIELDS = ('qpos', 'qvel', 'qacc', 'qacc_warmstart', 'qfrc_constraint', 'ncon', 'nefc', 'contact_pos',
          'contact_frame', 'contact_dist', 'contact_geom', 'efc_force', 'efc_state', 'osc_tau', 'ctrl')
REPLICAS = (0, 1, 2047, 4095)
CAPS = (1 << 9) | (1 << 10)   # Newton and line-search iteration caps: not errors


def _run(sc, nworld, acts, replicate):
    import torch
    from libero_hip import native
    from libero_hip.model import Model
    m = Model(sc)
    dm = native.DeviceModel(m)
    dd = native.DeviceData(dm, nworld)
    qpos = sc.init_qpos.copy()
    a0 = acts[0].copy()
    if replicate:
        for w in replicate:
            qpos[w] = sc.init_qpos[0]
            a0[w] = acts[0][0]
    dd['qpos'].copy_(torch.from_numpy(qpos))
    dd['osc_gains'].copy_(torch.from_numpy(np.tile(np.r_[sc.osc['kp'], sc.osc['kd']], (nworld, 1))))
    dd['osc_q0'].copy_(torch.from_numpy(np.tile(sc.osc['q0'], (nworld, 1))))
    dd['body_active'].fill_(1)
    dd.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    dd['osc_action'].copy_(torch.from_numpy(a0))
    dd.control_step(25, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    return m, {k: dd[k].cpu().numpy() for k in FIELDS + ('overflow',)}


def test_full_size_batch_independence(gpu_available):
    from libero_hip import scene as S
    nworld = 4096
    print('case c3 full size', nworld, flush=True)
    big = S.make_scene('c3', nworld, seed=0)
    acts = S.make_actions(nworld, 1, seed=2)
    m, out = _run(big, nworld, acts, REPLICAS)
    assert m.body_active is None
    assert not (out['overflow'][:, 0] & ~CAPS).any(), np.unique(out['overflow'][:, 0])
    for k, v in out.items():
        if v.dtype.kind == 'f':
            assert np.isfinite(v).all(), k
    assert out['ncon'][:, 0].min() > 0
    # the same world at four places of the batch: bit-identical
    for w in REPLICAS[1:]:
        for k in FIELDS:
            np.testing.assert_array_equal(out[k][w], out[k][REPLICAS[0]], err_msg='%s world %d' % (k, w))
    # and the same world in a batch of 16
    small = S.make_scene('c3', 16, seed=0)
    small.init_qpos[0] = big.init_qpos[0]
    sacts = S.make_actions(16, 1, seed=2)
    sacts[0][0] = acts[0][0]
    ms, sout = _run(small, 16, sacts, ())
    for k in ('geom_size', 'body_mass', 'dof_damping'):
        if k in m.arrays:
            np.testing.assert_array_equal(ms.arrays[k], m.arrays[k])
    for k in FIELDS:
        np.testing.assert_array_equal(sout[k][0], out[k][0], err_msg=k)
