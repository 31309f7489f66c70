"""CPU checks that pin the FP64 oracle (no GPU).

The oracle is the parity reference of the HIP control step, so it is checked here against data and
mathematics it does not share code with:

* FP64 OSC: golden vectors of tests/golden/osc_fixture.npz (numpy inv/pinv and robosuite's formulas,
  the recipe of the reference's tests/cuda/osc_reference_fixture.py:36-66);
* matrix helpers: numpy inverse / pseudo-inverse / SVD rank;
* mass matrix: kinetic-energy identity 1/2 qd'M qd = sum of body kinetic energies, the body
  velocities taken by central differences of forward kinematics;
* bias forces: Lagrange's equations, bias = Mdot qd - dT/dq + dV/dq, all three terms by
  central differences of the oracle's own M and body positions;
* site Jacobian: central differences of the site pose;
* Euler: MuJoCo's implicit-damping step in closed form and the quaternion exponential map;
* constraint forces: the Newton optimality condition M qacc = f_smooth + f_constraint, cone
  feasibility and, for free bodies, that the generalized constraint force equals the resultant of
  the published contact forces (an independent check of the contact Jacobian).
"""
import numpy as np
import pytest

from helpers import make_oracle
from libero_hip import scene as S
from libero_hip.model import Model, quat2mat
from oracle import oracle as O

GOLDEN = __import__('pathlib').Path(__file__).resolve().parent / 'golden'


# ------------------------------------------------------------------------------------ OSC
def test_osc_golden_fixture():
    f = np.load(GOLDEN / 'osc_fixture.npz')
    assert len(f['tau']) == 24
    for i in range(len(f['tau'])):
        inputs = dict(mass=f['pm'][i], jac=f['pj'][i], q=f['pq'][i], qvel=f['pv'][i], bias=f['bias'][i],
                      ee_pos=f['pp'][i], ee_rot=f['pr'][i], ee_vel=f['pe'][i])
        err, tau, ctrl, rank, *_ = O.osc(inputs, np.zeros(7), f['gains'][i], f['q0'][i], f['range'][i],
                                         f['goal_pos'][i], f['goal_rot'][i], np.zeros(2), policy=False)
        assert err == 0, i
        np.testing.assert_array_equal(rank, f['ranks'][i], err_msg='case %d' % i)
        ref = f['tau'][i]
        assert np.max(np.abs(tau - ref)) <= 1e-9 * max(np.max(np.abs(ref)), 1e-12), i
        # torques are clipped to the actuator range before they become controls
        np.testing.assert_allclose(ctrl[:7], np.clip(tau, -87, 87), rtol=0, atol=1e-12)


def test_osc_fixture_generator_is_deterministic(tmp_path):
    import importlib.util
    spec = importlib.util.spec_from_file_location('mk', GOLDEN / 'make_osc_fixture.py')
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    mk.main(tmp_path / 'f.npz')
    mk.main_ndof(tmp_path / 'g.npz')
    for fresh, name in ((tmp_path / 'f.npz', 'osc_fixture.npz'), (tmp_path / 'g.npz', 'osc_fixture_ndof.npz')):
        new, old = np.load(fresh), np.load(GOLDEN / name)
        for k in old.files:
            np.testing.assert_allclose(new[k], old[k], rtol=1e-12, atol=1e-14, err_msg=k)


def test_osc_other_joint_counts_golden_fixture():
    """Arms of 6 and 8 joints: the controller is sized by its joint count (numpy golden vectors)."""
    f = np.load(GOLDEN / 'osc_fixture_ndof.npz')
    assert sorted(set(f['ndof'].tolist())) == [6, 8]
    for i in range(len(f['tau'])):
        n = int(f['ndof'][i])
        inputs = dict(mass=f['pm'][i][:n * n], jac=f['pj'][i][:6 * n], q=f['pq'][i][:n], qvel=f['pv'][i][:n],
                      bias=f['bias'][i][:n], ee_pos=f['pp'][i], ee_rot=f['pr'][i], ee_vel=f['pe'][i])
        err, tau, ctrl, rank, *_ = O.osc(inputs, np.zeros(7), f['gains'][i], f['q0'][i][:n], f['range'][i][:2 * (n + 2)],
                                         f['goal_pos'][i], f['goal_rot'][i], np.zeros(2), policy=False)
        assert err == 0, i
        assert len(tau) == n and len(ctrl) == n + 2
        np.testing.assert_array_equal(rank, f['ranks'][i], err_msg='case %d' % i)
        ref = f['tau'][i][:n]
        assert np.max(np.abs(tau - ref)) <= 1e-9 * max(np.max(np.abs(ref)), 1e-12), i


def test_spd_inverse_matches_numpy():
    rng = np.random.default_rng(5)
    for n in (1, 3, 6, 7):
        a = rng.normal(size=(n, n))
        a = a @ a.T + n * np.eye(n)
        rc, inv = O.spd_inverse(a)
        assert rc == 0
        np.testing.assert_allclose(inv, np.linalg.inv(a), rtol=1e-11, atol=1e-13)


@pytest.mark.parametrize('rank', [0, 1, 2, 3, 5, 6])
def test_pinv_matches_numpy(rank):
    rng = np.random.default_rng(10 + rank)
    n = 6
    b = rng.normal(size=(n, rank))
    a = b @ b.T
    if rank == 0:
        a = np.zeros((n, n))
    ok, p, r = O.pinv(a)
    assert r == rank
    ref = np.linalg.pinv(a)
    np.testing.assert_allclose(p, ref, rtol=0, atol=1e-9 * max(np.max(np.abs(ref)), 1.0))


def test_pinv_ill_conditioned_uses_svd_rank():
    # condition number far above the Gauss-Jordan fast path's bound: rank from singular values
    u, _ = np.linalg.qr(np.random.default_rng(3).normal(size=(3, 3)))
    a = u @ np.diag([1.0, 1e-9, 1e-17]) @ u.T
    ok, p, r = O.pinv(a)
    s = np.linalg.svd(a, compute_uv=False)
    assert r == int(np.sum(s > 1e-15 * s.max()))
    np.testing.assert_allclose(p, np.linalg.pinv(a, rcond=1e-15), rtol=1e-6)


# ------------------------------------------------------------------------------------ dynamics
def _robot(nworld):
    m = Model(S.make_scene('c2', nworld, seed=3))
    om, od = make_oracle(m, nworld)
    return m, om, od


def _forward(od, qpos, qvel):
    od['qpos'][:] = qpos
    od['qvel'][:] = qvel
    od.forward(None, O_FLAGS)


O_FLAGS = 8 | 2   # bootstrap the controller goal, no control update


def dense_M(m, flat):
    a = m.arrays
    M = np.zeros((m.nv, m.nv))
    for t in range(m.ntree):
        adr, n, madr = int(a['tree_dofadr'][t]), int(a['tree_dofnum'][t]), int(a['tree_madr'][t])
        M[adr:adr + n, adr:adr + n] = flat[madr:madr + n * n].reshape(n, n)
    return M


def _body_frames(m, od, w):
    """World inertial frames (position of the centre of mass, rotation) of every body of world w."""
    a = m.arrays
    xpos = od['xpos'][w].reshape(-1, 3)
    xmat = od['xmat'][w].reshape(-1, 3, 3)
    ipos = a['body_ipos'].reshape(-1, 3)
    iquat = a['body_iquat'].reshape(-1, 4)
    com = xpos + np.einsum('bij,bj->bi', xmat, ipos)
    rot = np.stack([xmat[b] @ quat2mat(iquat[b]) for b in range(m.nbody)])
    return com, rot


def _kinetic_fd(m, od, wp, wm, w0, eps):
    """Sum of body kinetic energies from central differences between worlds wp and wm."""
    a = m.arrays
    cp, rp = _body_frames(m, od, wp)
    cm, rm = _body_frames(m, od, wm)
    _, r0 = _body_frames(m, od, w0)
    inertia = a['body_inertia'].reshape(-1, 3)
    ke = 0.0
    for b in range(1, m.nbody):
        v = (cp[b] - cm[b]) / (2 * eps)
        wx = ((rp[b] - rm[b]) / (2 * eps)) @ r0[b].T
        omega = np.array([wx[2, 1] - wx[1, 2], wx[0, 2] - wx[2, 0], wx[1, 0] - wx[0, 1]]) / 2
        ol = r0[b].T @ omega
        ke += 0.5 * a['body_mass'][b] * v @ v + 0.5 * ol @ (inertia[b] * ol)
    return ke


def test_mass_matrix_kinetic_energy_identity():
    m, om, od = _robot(3)
    rng = np.random.default_rng(11)
    q = m.scene.init_qpos[0] + rng.uniform(-0.4, 0.4, m.nq)
    qd = rng.uniform(-1, 1, m.nv)
    eps = 1e-6
    _forward(od, np.stack([q, q + eps * qd, q - eps * qd]), 0)
    M = dense_M(m, od['M'][0])
    np.testing.assert_allclose(M, M.T, rtol=0, atol=1e-14)
    assert np.all(np.linalg.eigvalsh(M) > 0)
    rigid = M - np.diag(m.arrays['dof_armature'])
    ke = _kinetic_fd(m, od, 1, 2, 0, eps)
    assert abs(0.5 * qd @ rigid @ qd - ke) <= 1e-7 * ke


def test_bias_forces_satisfy_lagrange_equations():
    m, om, od = _robot(3 + 2 * 9)
    nv = m.nv
    rng = np.random.default_rng(12)
    q = m.scene.init_qpos[0] + rng.uniform(-0.4, 0.4, m.nq)
    qd = rng.uniform(-1, 1, nv)
    eps = 1e-5
    qs = [q, q + eps * qd, q - eps * qd]
    for i in range(nv):
        e = np.zeros(nv)
        e[i] = eps
        qs += [q + e, q - e]
    qvel = np.zeros((len(qs), nv))
    qvel[0] = qd
    _forward(od, np.stack(qs), qvel)
    Ms = [dense_M(m, od['M'][w]) for w in range(len(qs))]
    bias = od['qfrc_bias'][0]
    mdot_qd = (Ms[1] - Ms[2]) @ qd / (2 * eps)
    g = np.array(m.opt.gravity, float)
    dT, dV = np.zeros(nv), np.zeros(nv)
    mass = m.arrays['body_mass']
    for i in range(nv):
        wp, wm = 3 + 2 * i, 4 + 2 * i
        dT[i] = 0.5 * qd @ (Ms[wp] - Ms[wm]) @ qd / (2 * eps)
        cp, _ = _body_frames(m, od, wp)
        cm, _ = _body_frames(m, od, wm)
        dV[i] = -np.sum(mass[:, None] * g[None, :] * (cp - cm)) / (2 * eps)
    expect = mdot_qd - dT + dV
    assert np.max(np.abs(bias - expect)) <= 1e-6 * np.max(np.abs(expect))


def test_site_jacobian_by_finite_differences():
    m, om, od = _robot(1 + 2 * 7)
    rng = np.random.default_rng(13)
    q = m.scene.init_qpos[0] + rng.uniform(-0.3, 0.3, m.nq)
    eps = 1e-6
    qs = [q]
    adr = m.arrays['osc_qposadr']
    for i in range(7):
        e = np.zeros(m.nq)
        e[adr[i]] = eps
        qs += [q + e, q - e]
    od['qpos'][:] = np.stack(qs)
    od.forward(None, 8)                   # run the controller so that it gathers its inputs
    jac = od['osc_jac'][0].reshape(6, 7)
    s = m.osc_site
    r0 = od['site_xmat'][0].reshape(-1, 3, 3)[s]
    for i in range(7):
        pp = od['site_xpos'][1 + 2 * i].reshape(-1, 3)[s]
        pm = od['site_xpos'][2 + 2 * i].reshape(-1, 3)[s]
        rp = od['site_xmat'][1 + 2 * i].reshape(-1, 3, 3)[s]
        rm = od['site_xmat'][2 + 2 * i].reshape(-1, 3, 3)[s]
        wx = (rp - rm) / (2 * eps) @ r0.T
        omega = np.array([wx[2, 1] - wx[1, 2], wx[0, 2] - wx[2, 0], wx[1, 0] - wx[0, 1]]) / 2
        np.testing.assert_allclose(jac[:3, i], (pp - pm) / (2 * eps), rtol=0, atol=1e-8)
        np.testing.assert_allclose(jac[3:, i], omega, rtol=0, atol=1e-8)


def test_gravity_bias_at_rest_is_potential_gradient():
    m, om, od = _robot(1 + 2 * 9)
    rng = np.random.default_rng(14)
    q = m.scene.init_qpos[0] + rng.uniform(-0.4, 0.4, m.nq)
    eps = 1e-6
    qs = [q]
    for i in range(m.nv):
        e = np.zeros(m.nq)
        e[i] = eps
        qs += [q + e, q - e]
    _forward(od, np.stack(qs), 0)
    mass = m.arrays['body_mass']
    g = np.array([0.0, 0.0, -9.81])
    dV = np.zeros(m.nv)
    for i in range(m.nv):
        cp, _ = _body_frames(m, od, 1 + 2 * i)
        cm, _ = _body_frames(m, od, 2 + 2 * i)
        dV[i] = -np.sum(mass[:, None] * g[None, :] * (cp - cm)) / (2 * eps)
    np.testing.assert_allclose(od['qfrc_bias'][0], dV, rtol=0, atol=1e-7 * np.max(np.abs(dV)))


def test_euler_implicit_damping_closed_form():
    m, om, od = _robot(2)
    rng = np.random.default_rng(15)
    q = m.scene.init_qpos[:2] + rng.uniform(-0.3, 0.3, (2, m.nq))
    qd = rng.uniform(-1, 1, (2, m.nv))
    _forward(od, q, qd)
    h = m.opt.timestep
    D = np.diag(m.arrays['dof_damping'])
    expect_v, expect_q = [], []
    for w in range(2):
        M = dense_M(m, od['M'][w])
        f = od['qfrc_smooth'][w] + od['qfrc_constraint'][w]
        v = qd[w] + h * np.linalg.solve(M + h * D, f)
        expect_v.append(v)
        expect_q.append(q[w] + h * v)      # hinge and slide joints only
    od['qpos'][:] = q
    od['qvel'][:] = qd
    od.control_step(1, 2)
    np.testing.assert_allclose(od['qvel'], np.array(expect_v), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(od['qpos'], np.array(expect_q), rtol=1e-12, atol=1e-12)


def test_free_joint_quaternion_exponential_map():
    m = Model(S.make_scene('c1', 1, seed=2))
    om, od = make_oracle(m, 1)
    q = m.scene.init_qpos[0].copy()
    q[:9] = m.scene.init_qpos[0][:9]
    rng = np.random.default_rng(16)
    qd = np.zeros(m.nv)
    jt = m.arrays['jnt_type']
    free = [j for j in range(m.njnt) if jt[j] == 0]
    j = free[0]
    qa, da = m.arrays['jnt_qposadr'][j], m.arrays['jnt_dofadr'][j]
    q[qa:qa + 3] += [0, 0, 0.5]          # lift clear of every contact
    qd[da + 3:da + 6] = rng.uniform(-3, 3, 3)
    od['qpos'][:] = q
    od['qvel'][:] = qd
    od.forward(None, O_FLAGS)
    h = m.opt.timestep
    od.control_step(1, 2)
    w = od['qvel'][0][da + 3:da + 6]      # angular velocity after the velocity update (local frame)
    angle = h * np.linalg.norm(w)
    axis = w / np.linalg.norm(w)
    dq = np.r_[np.cos(angle / 2), axis * np.sin(angle / 2)]
    q0 = q[qa + 3:qa + 7] / np.linalg.norm(q[qa + 3:qa + 7])
    a, b = q0, dq
    expect = np.array([a[0] * b[0] - a[1:] @ b[1:], *(a[0] * b[1:] + b[0] * a[1:] + np.cross(a[1:], b[1:]))])
    got = od['qpos'][0][qa + 3:qa + 7]
    np.testing.assert_allclose(got, expect, rtol=0, atol=1e-14)
    assert abs(np.linalg.norm(got) - 1) < 1e-14


# ------------------------------------------------------------------------------------ constraints
def _contact_forces_world(od, w, cone):
    """World-frame force on geom 2 of each contact from the published constraint rows."""
    ncon = int(od['ncon'][w, 0])
    nefc = int(od['nefc'][w, 0])
    frame = od['contact_frame'][w].reshape(-1, 3, 3)
    fric = od['contact_friction'][w].reshape(-1, 5)
    dim = od['contact_dim'][w]
    typ, cid, force = od['efc_type'][w][:nefc], od['efc_id'][w][:nefc], od['efc_force'][w][:nefc]
    out = np.zeros((ncon, 3))
    for c in range(ncon):
        rows = np.where((cid == c) & (typ >= 5))[0]
        f = force[rows]
        if cone == 1:                                    # elliptic: (normal, tangent...) rows
            local = np.zeros(3)
            local[:len(f)] = f[:3]
        else:                                            # pyramidal: edge pairs
            local = np.zeros(3)
            local[0] = f.sum()
            for j in range(min(2, (dim[c] - 1))):
                local[1 + j] = fric[c, j] * (f[2 * j] - f[2 * j + 1])
        out[c] = frame[c].T @ local
    return out


@pytest.mark.parametrize('config,cone', [('c1', 1), ('c3', 0)])
def test_newton_solution_is_optimal_and_consistent(config, cone):
    nworld = 2
    m = Model(S.make_scene(config, nworld, seed=4))
    assert m.opt.cone == cone
    om, od = make_oracle(m, nworld)
    od['qpos'][:] = m.scene.init_qpos[:nworld]
    od.forward(None, O_FLAGS)
    od.control_step(25, 2)                     # let the objects land on the table
    od.forward(None, O_FLAGS & ~8)
    a = m.arrays
    for w in range(nworld):
        ncon = int(od['ncon'][w, 0])
        assert ncon > 0
        M = dense_M(m, od['M'][w])
        resid = M @ od['qacc'][w] - od['qfrc_smooth'][w] - od['qfrc_constraint'][w]
        scale = np.max(np.abs(od['qfrc_smooth'][w])) + np.max(np.abs(od['qfrc_constraint'][w]))
        assert np.max(np.abs(resid)) <= 1e-6 * scale, config
        nefc = int(od['nefc'][w, 0])
        typ, force = od['efc_type'][w][:nefc], od['efc_force'][w][:nefc]
        if cone == 0:
            assert np.all(force[typ == 6] >= -1e-12)
        else:
            cid = od['efc_id'][w][:nefc]
            fric = od['contact_friction'][w].reshape(-1, 5)
            for c in range(ncon):
                f = force[(cid == c) & (typ == 7)]
                assert f[0] >= -1e-12
                mu = fric[c, :len(f) - 1]
                assert np.linalg.norm(f[1:] / np.maximum(mu, 1e-30)) <= f[0] * (1 + 1e-6) + 1e-9
        # free bodies: generalized constraint force = resultant of the contact forces (world frame)
        fw = _contact_forces_world(od, w, cone)
        geom_body = a['geom_body']
        cg = od['contact_geom'][w].reshape(-1, 2)
        for j in range(m.njnt):
            if a['jnt_type'][j] != 0:
                continue
            body, da = a['jnt_body'][j], a['jnt_dofadr'][j]
            total = np.zeros(3)
            torque = np.zeros(3)
            anchor = od['xpos'][w].reshape(-1, 3)[body]
            pos = od['contact_pos'][w].reshape(-1, 3)
            for c in range(ncon):
                sign = int(geom_body[cg[c, 1]] == body) - int(geom_body[cg[c, 0]] == body)
                total += sign * fw[c]
                torque += sign * np.cross(pos[c] - anchor, fw[c])
            qc = od['qfrc_constraint'][w][da:da + 6]
            R = od['xmat'][w].reshape(-1, 3, 3)[body]
            tol = 1e-6 * max(np.max(np.abs(qc)), 1e-3)
            np.testing.assert_allclose(qc[:3], total, rtol=0, atol=tol)
            np.testing.assert_allclose(qc[3:], R.T @ torque, rtol=0, atol=tol)
