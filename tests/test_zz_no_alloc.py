"""mx_control_step_noalloc (no allocation; workspace slabs in the library's fixed device scratch)
against mx_control_step with the caller's workspace, through the C ABI.

Both entry points run the same kernels on the same inputs, so every output must be bit-identical.
Two calls in a row per model, the second on a smaller batch, so the second runs on scratch that
still holds the first call's slabs.  C3 runs on the workspace route by default; C4's working set
exceeds LDS, so its worlds need the slabs.  A batch beyond the scratch is refused before any
launch (host-only check).
"""
import ctypes as ct

import numpy as np
import pytest

from libero_hip import native, scene as S
from libero_hip.model import Model

STATE = ('qpos', 'qvel', 'qacc_warmstart', 'ctrl', 'time', 'osc_goal_pos', 'osc_goal_rot', 'osc_gripper',
         'osc_gains', 'osc_q0', 'osc_tau', 'osc_rank', 'osc_error', 'body_active')
OUTPUTS = STATE + ('qacc', 'qacc_smooth', 'qfrc_constraint', 'qfrc_bias', 'actuator_force', 'xpos', 'xquat',
                   'geom_xpos', 'site_xpos', 'ncon', 'nefc', 'solver_niter', 'contact_pos', 'contact_frame',
                   'contact_dist', 'contact_geom', 'efc_force', 'efc_pos', 'efc_D', 'efc_aref', 'efc_type',
                   'efc_state', 'efc_id', 'overflow', 'nstep')


def _state_of(m, sc, dm, n):
    """Scene initial state of n worlds, bootstrapped (OSC goal at the current pose) on the device."""
    import torch
    dd = native.DeviceData(dm, n)
    dd['qpos'].copy_(torch.from_numpy(sc.init_qpos[:n]))
    dd['osc_gains'].copy_(torch.from_numpy(np.tile(np.r_[sc.osc['kp'], sc.osc['kd']], (n, 1))))
    dd['osc_q0'].copy_(torch.from_numpy(np.tile(sc.osc['q0'], (n, 1))))
    if m.body_active is None:
        dd['body_active'].fill_(1)
    else:
        dd['body_active'].copy_(torch.from_numpy(m.body_active[:n]))
    dd.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    torch.cuda.synchronize()
    return {k: dd[k].clone() for k in STATE}


@pytest.mark.gpu
@pytest.mark.parametrize('config,sizes', [('c3', (96, 24)), ('c4', (6, 2))])
def test_noalloc_matches_workspace_entry(gpu_available, config, sizes):
    import torch
    sc = S.make_scene(config, sizes[0], seed=3)
    m = Model(sc)
    dm = native.DeviceModel(m)
    state = _state_of(m, sc, dm, sizes[0])
    acts = torch.from_numpy(S.make_actions(sizes[0], len(sizes), seed=4)).to('cuda')
    for call, n in enumerate(sizes):
        print('case', config, 'call', call, 'nworld', n, flush=True)
        a = native.DeviceData(dm, n)                                  # the caller's workspace
        b = native.DeviceData(dm, n, workspace=False, validate=False)  # none: the library's scratch
        assert a['workspace'].shape[1] > 1 and b['workspace'].shape[1] == 1
        for dd in (a, b):
            for k, v in state.items():
                dd[k].copy_(v[:n])
            dd['osc_action'].copy_(acts[call][:n])
        a.control_step(25, native.FLAG_POLICY_FIRST)
        b.control_step_noalloc(25, native.FLAG_POLICY_FIRST)
        torch.cuda.synchronize()
        ovf = a['overflow'].cpu().numpy()
        assert not (ovf & ~((1 << 9) | (1 << 10))).any()
        assert int(a['ncon'].cpu().numpy().max()) > 0
        for k in OUTPUTS:
            x, y = a[k].cpu().numpy(), b[k].cpu().numpy()
            assert np.array_equal(x, y, equal_nan=True), (config, call, k, np.abs(x - y).max())
        state = {k: a[k].clone() for k in STATE}


@pytest.mark.gpu
def test_noalloc_inside_a_captured_graph(gpu_available):
    """The use the header names: mx_control_step_noalloc captured into a HIP graph (torch.cuda.graph)
    and replayed.  Each replay starts from the same state, restored by eager copies between replays,
    and must equal an eager mx_control_step from that state bit for bit, replay after replay.  The
    first call on the device is made eagerly before the capture (it resolves the scratch address)."""
    import torch
    n = 24
    sc = S.make_scene('c3', n, seed=5)
    m = Model(sc)
    dm = native.DeviceModel(m)
    state = _state_of(m, sc, dm, n)
    acts = torch.from_numpy(S.make_actions(n, 1, seed=6)[0]).to('cuda')
    a = native.DeviceData(dm, n)
    b = native.DeviceData(dm, n, workspace=False, validate=False)

    def restore(dd):
        for k, v in state.items():
            dd[k].copy_(v)
        dd['osc_action'].copy_(acts)
        dd['nstep'].zero_()                 # counters the launches accumulate
        dd['overflow'].zero_()

    restore(a)
    a.control_step(25, native.FLAG_POLICY_FIRST)
    restore(b)
    b.control_step_noalloc(25, native.FLAG_POLICY_FIRST)          # eager first call on this device
    torch.cuda.synchronize()
    expect = {k: a[k].cpu().numpy() for k in OUTPUTS}
    assert int(expect['ncon'].max()) > 0
    for k in OUTPUTS:
        assert np.array_equal(expect[k], b[k].cpu().numpy(), equal_nan=True), ('eager', k)
    side = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    restore(b)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            b.control_step_noalloc(25, native.FLAG_POLICY_FIRST)
    torch.cuda.synchronize()
    for replay in range(3):
        print('replay', replay, flush=True)
        restore(b)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in OUTPUTS:
            y = b[k].cpu().numpy()
            assert np.array_equal(expect[k], y, equal_nan=True), (replay, k)
        restore(a)                                                # eager work between the replays
        a.control_step(25, native.FLAG_POLICY_FIRST)
        torch.cuda.synchronize()
    del g


def test_noalloc_refuses_a_batch_beyond_the_scratch():
    """(nworld + 1) slabs beyond MX_SCRATCH_BYTES: MX_ERR_SCRATCH before any device call."""
    from test_abi_host import HostModel
    lib = native.load()
    m = Model(S.make_scene('c3', 2))
    h = HostModel(m)
    slab = lib.mx_workspace_bytes(ct.byref(h.m))
    fits = native.SCRATCH_BYTES // slab - 1
    h.d.nworld = fits + 1
    assert lib.mx_control_step_noalloc(ct.byref(h.m), ct.byref(h.d), 25, 1, None) == native.ERR_SCRATCH
    assert 'scratch' in lib.mx_error_string(native.ERR_SCRATCH).decode()
