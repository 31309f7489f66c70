"""The workspace route at the configurations' full sizes (C3 N = 4096, C4 N = 8192, C5 N = 16384),
through properties that do not depend on the batch size.

The oracle is too slow to follow thousands of worlds, and the parity tests check the physics on
small batches; what changes with the batch size is the addressing (high world indices into the
workspace slabs, the shared image slab, a full grid of resident worlds, C5's 2 GB of slabs).  So,
at each full size:

* worlds given the same state and actions end one control step bit-identical wherever they sit in
  the batch (first, middle, last slab), and bit-identical to the same world run in a batch of 16;
* no overflow bit beyond the Newton / line-search iteration caps, every field finite;
* every world touches something (homogeneous batches rest objects on the table; in the
  heterogeneous C5 batch some worlds hold no object).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FIELDS = ('qpos', 'qvel', 'qacc', 'qacc_warmstart', 'qfrc_constraint', 'ncon', 'nefc', 'contact_pos',
          'contact_frame', 'contact_dist', 'contact_geom', 'efc_force', 'efc_state', 'osc_tau', 'ctrl')
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
    active = np.ones((nworld, m.nbody), np.int32) if m.body_active is None else m.body_active.copy()
    for w in replicate:
        qpos[w] = sc.init_qpos[0]
        a0[w] = acts[0][0]
        active[w] = active[0]
    dd['qpos'].copy_(torch.from_numpy(qpos))
    dd['osc_gains'].copy_(torch.from_numpy(np.tile(np.r_[sc.osc['kp'], sc.osc['kd']], (nworld, 1))))
    dd['osc_q0'].copy_(torch.from_numpy(np.tile(sc.osc['q0'], (nworld, 1))))
    dd['body_active'].copy_(torch.from_numpy(active))
    dd.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    dd['osc_action'].copy_(torch.from_numpy(a0))
    dd.control_step(25, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    return m, {k: dd[k].cpu().numpy() for k in FIELDS + ('overflow',)}


@pytest.mark.parametrize('config,nworld', [('c3', 4096), ('c4', 8192), ('c5', 16384)])
def test_full_size_batch_independence(gpu_available, config, nworld):
    from libero_hip import scene as S
    replicas = (0, 1, nworld // 2 - 1, nworld - 1)
    print('case %s full size' % config, nworld, flush=True)
    big = S.make_scene(config, nworld, seed=0)
    acts = S.make_actions(nworld, 1, seed=2)
    m, out = _run(big, nworld, acts, replicas)
    assert not (out['overflow'][:, 0] & ~CAPS).any(), np.unique(out['overflow'][:, 0])
    for k, v in out.items():
        if v.dtype.kind == 'f':
            assert np.isfinite(v).all(), k
    ncon = out['ncon'][:, 0]
    assert (ncon.min() if m.body_active is None else ncon.max()) > 0
    # the same world at four places of the batch: bit-identical
    for w in replicas[1:]:
        for k in FIELDS:
            np.testing.assert_array_equal(out[k][w], out[k][replicas[0]], err_msg='%s world %d' % (k, w))
    # and the same world in a batch of 16
    small = S.make_scene(config, 16, seed=0)
    small.init_qpos[0] = big.init_qpos[0]
    sacts = S.make_actions(16, 1, seed=2)
    sacts[0][0] = acts[0][0]
    ms, sout = _run(small, 16, sacts, ())
    for k in ('geom_size', 'body_mass', 'dof_damping'):
        if k in m.arrays:
            np.testing.assert_array_equal(ms.arrays[k], m.arrays[k])
    for k in FIELDS:
        np.testing.assert_array_equal(sout[k][0], out[k][0], err_msg=k)
