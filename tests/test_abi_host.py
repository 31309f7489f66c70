"""Host-side checks of the C-ABI library and the model compiler (no GPU call is made).

* libmx_physics.so loads, exports every entry point include/mx_physics.h declares, and agrees
  with the Python mirror on ABI version, struct sizes and field tables;
* mx_check admits the shipped configurations and rejects malformed or out-of-domain models with
  the documented error codes; mx_lds_bytes fits the 160 KiB LDS of one CU;
* the model compiler's invariants: DFS preorder subtrees, mass-matrix tree blocks, the collision
  pair filters, M(qpos0) against the oracle, and meaninertia.
"""
import ctypes as ct
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from libero_hip import layout, native, scene as S
from libero_hip.model import Model

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'mx_physics.h'


def declared_entry_points():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'^[a-z_ ]+[ *]+(mx_[a-z0-9_]+)\(', text, flags=re.M)))


def test_library_exports_every_declared_entry_point():
    lib = native.load()
    names = declared_entry_points()
    assert 'mx_control_step' in names and 'mx_forward' in names
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(native.EXPORTS) == names


def test_abi_identity():
    lib = native.load()
    assert lib.mx_abi_version() == layout.ABI_VERSION
    assert lib.mx_model_bytes() == ct.sizeof(native.MxModel)
    assert lib.mx_data_bytes() == ct.sizeof(native.MxData)
    assert lib.mx_arch() == 950
    assert lib.mx_source_id().decode().startswith('mx_step.hip')
    assert lib.mx_field_count(7) == -1 and lib.mx_field_name(0, 10 ** 6) is None
    for code, text in ((0, 'success'), (-1, 'invalid argument'), (-2, 'model outside the admitted domain'),
                       (-3, 'per-world working set exceeds the LDS budget and no (or too small a) workspace is given')):
        assert lib.mx_error_string(code).decode() == text


class HostModel:
    """MxModel / MxData filled with host buffers (valid for mx_check and mx_lds_bytes only)."""

    def __init__(self, model, nworld=2, workspace_doubles=0):
        self._keep = []
        s = native.MxModel()
        for k, v in layout.model_scalars(model).items():
            setattr(s, k, v)
        real, ints = layout.model_arrays(model)
        for name, arr in real.items():
            a = np.ascontiguousarray(arr, np.float32) if len(arr) else np.zeros(1, np.float32)
            self._keep.append(a)
            setattr(s, name, a.ctypes.data_as(ct.POINTER(ct.c_float)))
        for name, arr in ints.items():
            a = np.ascontiguousarray(arr, np.int32) if len(arr) else np.zeros(1, np.int32)
            self._keep.append(a)
            setattr(s, name, a.ctypes.data_as(ct.POINTER(ct.c_int32)))
        d = native.MxData()
        d.nworld = nworld
        d.workspace_doubles = workspace_doubles
        d.workspace_total = (nworld + 1) * workspace_doubles
        widths = layout.data_widths(model, workspace_doubles)
        for name in layout.DATA_REAL_ARRAYS:
            a = np.zeros(nworld * max(widths[name], 1), np.float32)
            self._keep.append(a)
            setattr(d, name, a.ctypes.data_as(ct.POINTER(ct.c_float)))
        for name in layout.DATA_F64_ARRAYS:
            rows = nworld + 1 if name == 'workspace' else nworld
            a = np.zeros(rows * max(widths[name], 1), np.float64)
            self._keep.append(a)
            setattr(d, name, a.ctypes.data_as(ct.POINTER(ct.c_double)))
        for name in layout.DATA_INT_ARRAYS:
            a = np.zeros(nworld * max(widths[name], 1), np.int32)
            self._keep.append(a)
            setattr(d, name, a.ctypes.data_as(ct.POINTER(ct.c_int32)))
        self.m, self.d = s, d

    def check(self):
        return native.load().mx_check(ct.byref(self.m), ct.byref(self.d))


@pytest.mark.parametrize('config', ['c1', 'c2', 'c3', 'c5'])
def test_check_admits_shipped_configs(config):
    h = HostModel(Model(S.make_scene(config, 2)))
    assert h.check() == 0
    lds = native.load().mx_lds_bytes(ct.byref(h.m))
    assert 0 < lds <= 160 * 1024


def test_workspace_route_admission():
    """The dense-clutter scene (C4) exceeds the LDS of a workgroup: it is admitted only with a
    workspace of at least mx_workspace_bytes per world, in whole 256-byte units."""
    lib = native.load()
    m = Model(S.make_scene('c4', 2))
    h = HostModel(m)
    lds = lib.mx_lds_bytes(ct.byref(h.m))
    ws = lib.mx_workspace_bytes(ct.byref(h.m))
    assert lds > layout.LDS_BUDGET and ws >= lds and ws % 256 == 0
    assert h.check() == -3                                  # no workspace
    assert HostModel(m, workspace_doubles=ws // 8).check() == 0
    assert HostModel(m, workspace_doubles=ws // 8 - 32).check() == -3    # too small
    assert HostModel(m, workspace_doubles=ws // 8 + 8).check() == -3     # slabs not 256-byte aligned
    h = HostModel(m, workspace_doubles=ws // 8)
    h.d.workspace_total -= 1                                # no room for the image slab
    assert h.check() == -3
    small = Model(S.make_scene('c3', 2))
    hs = HostModel(small)
    assert lib.mx_workspace_bytes(ct.byref(hs.m)) >= lib.mx_lds_bytes(ct.byref(hs.m))
    assert hs.check() == 0                                  # fits LDS: no workspace needed


def test_check_rejects_bad_models():
    lib = native.load()
    m = Model(S.make_scene('c1', 2))
    assert lib.mx_check(None, None) == -1
    h = HostModel(m)
    h.m.abi_version = 0
    assert h.check() == -1
    h = HostModel(m)
    h.d.nworld = 0
    assert h.check() == -1
    h = HostModel(m)
    h.m.njmax = 20000                   # above the row budget of the world-local solver
    assert h.check() == -2
    h = HostModel(m)
    h.m.ntree = 300                     # island ids are 8-bit
    assert h.check() == -2
    h = HostModel(m)
    h.m.njmax = 0                       # constraints enabled but no row capacity
    assert h.check() == -2
    h = HostModel(m)
    h.d.qpos = ct.POINTER(ct.c_float)()
    assert h.check() == -1
    h = HostModel(m)
    h.m.body_parent = ct.POINTER(ct.c_int32)()
    assert h.check() == -1


@pytest.mark.parametrize('name', [n for n in layout.MODEL_REAL_ARRAYS + layout.MODEL_INT_ARRAYS])
def test_check_rejects_null_model_array(name):
    """Every model array the kernels may index is checked before a launch (C callers get
    MX_ERR_INVALID instead of a device memory fault)."""
    h = HostModel(Model(S.make_scene('c3', 2)))
    assert h.check() == 0
    ctype = ct.c_float if name in layout.MODEL_REAL_ARRAYS else ct.c_int32
    setattr(h.m, name, ct.POINTER(ctype)())
    assert h.check() == -1


ROW_ARRAYS = ['ncon', 'nefc', 'solver_niter', 'contact_pos', 'contact_frame', 'contact_dist', 'contact_friction',
              'contact_includemargin', 'contact_geom', 'contact_dim', 'efc_force', 'efc_pos', 'efc_D', 'efc_aref',
              'efc_type', 'efc_state', 'efc_id']


@pytest.mark.parametrize('name', ROW_ARRAYS + ['body_active'])
def test_check_rejects_null_row_arrays(name):
    """Models with constraint rows publish contacts, rows and counts: those pointers must be set;
    body_active must be set for heterogeneous batches.  Smooth-only models need neither."""
    config = 'c5' if name == 'body_active' else 'c3'
    h = HostModel(Model(S.make_scene(config, 2)))
    ctype = ct.c_int32 if name in layout.DATA_INT_ARRAYS else ct.c_float
    setattr(h.d, name, ct.POINTER(ctype)())
    assert h.check() == -1
    smooth = HostModel(Model(S.make_scene('c2', 2)))
    setattr(smooth.d, name, ct.POINTER(ctype)())
    assert smooth.check() == 0


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / 'bench.py'), '--gpus', '2'], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert 'one GPU' in r.stdout + r.stderr


# ------------------------------------------------------------------------------ model compiler
@pytest.mark.parametrize('config', ['c1', 'c2', 'c3', 'c4', 'c5'])
def test_model_compiler_invariants(config):
    m = Model(S.make_scene(config, 2))
    a = m.arrays
    parent = a['body_parent']
    size = a['body_subtreesize']
    for b in range(1, m.nbody):
        p = parent[b]
        assert p < b < p + size[p]                      # DFS preorder: contiguous subtrees
    # tree blocks tile the dofs and the dense M storage
    adr = 0
    for t in range(m.ntree):
        assert a['tree_dofadr'][t] == sum(a['tree_dofnum'][:t])
        assert a['tree_madr'][t] == adr
        adr += a['tree_dofnum'][t] ** 2
    assert adr == m.nM
    # collision pairs: never the same body or a parent-child pair, no duplicates
    gb = a['geom_body']
    pairs = a['pair_geom'].reshape(-1, 2)
    seen = set()
    for g1, g2 in pairs:
        b1, b2 = gb[g1], gb[g2]
        assert b1 != b2
        assert not (b1 > 0 and b2 > 0 and (parent[b1] == b2 or parent[b2] == b1))
        assert a['geom_type'][g1] <= a['geom_type'][g2]
        assert (g1, g2) not in seen
        seen.add((g1, g2))
    assert m.meaninertia > 0 and np.all(a['body_invweight0'] >= 0)


def test_mass_matrix_at_qpos0_matches_oracle():
    from helpers import make_oracle
    m = Model(S.make_scene('c1', 1))
    om, od = make_oracle(m, 1)
    od['qpos'][:] = a = m.arrays['qpos0']
    od.forward(None, 8 | 2)
    M = np.zeros((m.nv, m.nv))
    ar = m.arrays
    for t in range(m.ntree):
        d0, n, madr = int(ar['tree_dofadr'][t]), int(ar['tree_dofnum'][t]), int(ar['tree_madr'][t])
        M[d0:d0 + n, d0:d0 + n] = od['M'][0][madr:madr + n * n].reshape(n, n)
    assert abs(np.mean(np.diag(M)) - m.meaninertia) <= 1e-12 * m.meaninertia
    assert a.shape == (m.nq,)


def test_model_compiler_rejects_unsupported_condim():
    sc = S.make_scene('c1', 2)
    for b in sc.bodies:
        for g in getattr(b, 'geoms', []):
            g.condim = 6
            break
    with pytest.raises(ValueError, match='condim'):
        Model(sc)
