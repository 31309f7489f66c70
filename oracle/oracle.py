"""ctypes binding of the CPU FP64 oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.  It
packs a compiled model into the oracle's double-precision ``OrModel`` (same field tables as the
device ``MxModel``) and holds host ``OrData`` buffers for ``nworld`` worlds.
"""
from __future__ import annotations

import ctypes as ct
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
sys.path.insert(0, str(ROOT / 'gpu-libero_amd'))
from libero_hip import layout  # noqa: E402

LIB_PATH = HERE / 'liboracle.so'


def build(force=False):
    """Compile the oracle with its Makefile (g++ only)."""
    if force or not LIB_PATH.exists():
        subprocess.run(['make', '-s', '-C', str(HERE)] + (['-B'] if force else []), check=True)
    return LIB_PATH


_LIB = None


def library():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        lib = ct.CDLL(str(LIB_PATH))
        lib.or_field_count.restype = ct.c_int
        lib.or_field_name.restype = ct.c_char_p
        lib.or_field_name.argtypes = [ct.c_int, ct.c_int]
        lib.or_model_bytes.restype = ct.c_size_t
        lib.or_data_bytes.restype = ct.c_size_t
        layout.check_field_tables(lib.or_field_count, lib.or_field_name, 'oracle')
        lib.or_control_step.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int, ct.c_int, ct.c_int]
        lib.or_forward.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int]
        dp = ct.POINTER(ct.c_double)
        ip = ct.POINTER(ct.c_int32)
        lib.or_osc.argtypes = [ct.c_int] + [dp] * 13 + [ct.c_int, ct.c_double, ct.c_int] + [dp] * 5 + [ip]
        lib.or_spd_inverse.argtypes = [dp, ct.c_int, dp]
        lib.or_pinv.argtypes = [dp, ct.c_int, dp, ip]
        _LIB = lib
    return _LIB


OrModel = layout.make_struct('OrModel', ct.c_double, ct.c_double, 'model')
OrData = layout.make_struct('OrData', ct.c_double, ct.c_double, 'data')


def _ptr(arr, ctype):
    return arr.ctypes.data_as(ct.POINTER(ctype))


class OracleModel:
    def __init__(self, model, fp32_model=False):
        """fp32_model: the model's real scalars and arrays rounded to float32 first (the values the
        device's FP32 model arena holds), for comparing the device's FP64 route at tolerances below
        the rounding of the model itself."""
        lib = library()
        if ct.sizeof(OrModel) != lib.or_model_bytes() or ct.sizeof(OrData) != lib.or_data_bytes():
            raise ImportError('oracle struct sizes differ from the Python mirror')
        self.model = model
        real, ints = layout.model_arrays(model)
        self._keep = []
        s = OrModel()
        for k, v in layout.model_scalars(model).items():
            if fp32_model and k in layout.MODEL_REAL_SCALARS:
                v = float(np.float32(v))
            setattr(s, k, v)
        for name, arr in real.items():
            arr = np.ascontiguousarray(arr, np.float64) if len(arr) else np.zeros(1)
            if fp32_model:
                arr = arr.astype(np.float32).astype(np.float64)
            self._keep.append(arr)
            setattr(s, name, _ptr(arr, ct.c_double))
        for name, arr in ints.items():
            arr = np.ascontiguousarray(arr, np.int32) if len(arr) else np.zeros(1, np.int32)
            self._keep.append(arr)
            setattr(s, name, _ptr(arr, ct.c_int32))
        self.struct = s


class OracleData:
    """Host double-precision per-world buffers, world-major ``(nworld, width)``."""

    def __init__(self, omodel, nworld):
        self.omodel = omodel
        m = omodel.model
        widths = layout.data_widths(m)
        self.nworld = nworld
        self.arrays = {}
        s = OrData()
        s.nworld = nworld
        for name in layout.DATA_REAL_ARRAYS + layout.DATA_F64_ARRAYS:
            arr = np.zeros((nworld, max(widths[name], 1)), np.float64)
            self.arrays[name] = arr
            setattr(s, name, _ptr(arr, ct.c_double))
        for name in layout.DATA_INT_ARRAYS:
            arr = np.zeros((nworld, max(widths[name], 1)), np.int32)
            self.arrays[name] = arr
            setattr(s, name, _ptr(arr, ct.c_int32))
        self.struct = s
        self.arrays['osc_action_scale'][:] = m.osc_action_scale

    def __getitem__(self, name):
        return self.arrays[name]

    def control_step(self, substeps, flags, threads=1, pin=False):
        rc = library().or_control_step(ct.byref(self.omodel.struct), ct.byref(self.struct),
                                       substeps, flags, threads, int(pin))
        if rc:
            raise RuntimeError('oracle control step failed: %d' % rc)

    def forward(self, mask=None, flags=0, threads=1):
        m = None if mask is None else np.ascontiguousarray(mask, np.int32)
        rc = library().or_forward(ct.byref(self.omodel.struct), ct.byref(self.struct),
                                  None if m is None else m.ctypes.data, flags, threads)
        if rc:
            raise RuntimeError('oracle forward failed: %d' % rc)


def osc(inputs, action, gains, q0, ctrlrange, goal_pos, goal_rot, gripper, *, policy, uncouple=1,
        speed=0.01, action_scale=None):
    """Run the FP64 OSC alone on n arm joints (n from the size of inputs['q']); returns (error, tau,
    ctrl, rank, goal_pos, goal_rot, gripper).  action_scale: robosuite's input_min, input_max,
    output_min, output_max (24 values) or None for OSC_POSE's default ranges."""
    lib = library()
    n = int(np.asarray(inputs['q']).size)
    d = lambda x, k: np.ascontiguousarray(np.asarray(x, np.float64).reshape(-1)[:k])  # noqa: E731
    args = [d(inputs['mass'], n * n), d(inputs['jac'], 6 * n), d(inputs['q'], n), d(inputs['qvel'], n),
            d(inputs['bias'], n), d(inputs['ee_pos'], 3), d(inputs['ee_rot'], 9), d(inputs['ee_vel'], 6),
            d(action, 7)]
    scale = None if action_scale is None else d(action_scale, 24)
    rest = [d(gains, 12), d(q0, n), d(ctrlrange, 2 * (n + 2))]
    gp, gr, gg = d(goal_pos, 3).copy(), d(goal_rot, 9).copy(), d(gripper, 2).copy()
    tau, ctrl, rank = np.zeros(n), np.zeros(n + 2), np.zeros(3, np.int32)
    err = lib.or_osc(n, *[_ptr(a, ct.c_double) for a in args], None if scale is None else _ptr(scale, ct.c_double),
                     *[_ptr(a, ct.c_double) for a in rest], uncouple, speed, int(policy),
                     _ptr(gp, ct.c_double), _ptr(gr, ct.c_double), _ptr(gg, ct.c_double),
                     _ptr(tau, ct.c_double), _ptr(ctrl, ct.c_double), _ptr(rank, ct.c_int32))
    return err, tau, ctrl, rank, gp, gr, gg


def spd_inverse(a):
    a = np.ascontiguousarray(a, np.float64)
    out = np.zeros_like(a)
    rc = library().or_spd_inverse(_ptr(a, ct.c_double), a.shape[0], _ptr(out, ct.c_double))
    return rc, out


def pinv(a):
    a = np.ascontiguousarray(a, np.float64)
    out = np.zeros_like(a)
    rank = np.zeros(1, np.int32)
    ok = library().or_pinv(_ptr(a, ct.c_double), a.shape[0], _ptr(out, ct.c_double), _ptr(rank, ct.c_int32))
    return ok, out, int(rank[0])


def contact_frame(normal):
    """The 3 x 3 contact frame (rows: normal, tangent, normal x tangent) the step builds for a
    contact normal."""
    n = np.ascontiguousarray(np.asarray(normal, np.float64).reshape(3))
    out = np.zeros(9)
    library().or_contact_frame(_ptr(n, ct.c_double), _ptr(out, ct.c_double))
    return out.reshape(3, 3)


def set_horizon_capacity(capacity=24):
    """EPA horizon edge capacity of the oracle's polytope (24, the device's; tests shrink it)."""
    library().or_set_horizon_capacity(int(capacity))


def last_collide_flags():
    """Overflow bits of the last collide() call on this thread (MX_OVERFLOW_EPA_HORIZON = 1 << 8)."""
    lib = library()
    lib.or_last_collide_flags.restype = ct.c_int
    return int(lib.or_last_collide_flags())


_HULLS = {}   # hull polygon packs by vertex bytes (tests call collide on the same hulls many times)


def collide(g1, g2, margin=0.0, maxout=8, *, gap=0.0, boxbox='primitive', tolerance=1e-6, iterations=35,
            epa_iterations=None, convex='gjk'):
    """Oracle narrowphase on two geom dicts {type, pos, mat(3x3), size, vert}; returns (pos, normal, dist).

    ``boxbox`` selects the box-box route: 'primitive' (SAT and face clipping) or 'convex' (GJK/EPA and
    the box manifold); EPA runs ``epa_iterations`` (default: 16 for box-box, else ``iterations``).
    ``convex='mpr'`` takes convex pairs through MPR (MuJoCo 2.3.7) with ``tolerance`` and
    ``iterations`` as its mpr_tolerance and mpr_iterations and the zero tests of the reference's FP32
    route (FLT_EPSILON); ``convex='mpr64'`` the same with those of MuJoCo's double build."""
    lib = library()
    lib.or_collide.restype = ct.c_int

    def parts(g):
        pos = np.ascontiguousarray(np.asarray(g['pos'], np.float64).reshape(3))
        mat = np.ascontiguousarray(np.asarray(g.get('mat', np.eye(3)), np.float64).reshape(9))
        size = np.ascontiguousarray(np.asarray(list(g.get('size', (0, 0, 0))) + [0, 0, 0], np.float64)[:3])
        vert = np.ascontiguousarray(np.asarray(g.get('vert', np.zeros((1, 3))), np.float64).reshape(-1))
        nv = 0 if 'vert' not in g else len(vert) // 3
        pack, norms = None, None
        if nv and vert.tobytes() in _HULLS:
            pack, norms = _HULLS[vert.tobytes()]
        elif nv:   # the hull polygons, as the model compiler builds them
            from libero_hip.model import mesh_polygons
            polys = mesh_polygons(vert.reshape(-1, 3))
            inc = [[] for _ in range(nv)]
            for pid, (ids, _) in enumerate(polys):
                for i in ids:
                    inc[i].append(pid)
            lens = [len(p[0]) for p in polys]
            vadr = np.concatenate([[0], np.cumsum(lens)[:-1]])
            madr = np.concatenate([[0], np.cumsum([len(x) for x in inc])[:-1]])
            pack = np.ascontiguousarray(np.concatenate(
                [[len(polys), nv], vadr, lens, madr, [len(x) for x in inc],
                 [i for p in polys for i in p[0]], [k for x in inc for k in x]]).astype(np.int32))
            norms = np.ascontiguousarray(np.array([p[1] for p in polys], np.float64).reshape(-1))
            if len(_HULLS) < 256:
                _HULLS[vert.tobytes()] = pack, norms
        return pos, mat, size, vert, nv, pack, norms

    p1, m1, s1, v1, n1, q1, r1 = parts(g1)
    p2, m2, s2, v2, n2, q2, r2 = parts(g2)
    ip = lambda a: None if a is None else _ptr(a, ct.c_int32)  # noqa: E731
    np_ = lambda a: None if a is None else _ptr(a, ct.c_double)  # noqa: E731
    op, on, od = np.zeros(3 * maxout), np.zeros(3 * maxout), np.zeros(maxout)
    dp = lambda a: _ptr(a, ct.c_double)  # noqa: E731
    if epa_iterations is None:
        epa_iterations = 16 if int(g1['type']) == 6 and int(g2['type']) == 6 else iterations
    n = lib.or_collide(int(g1['type']), dp(p1), dp(m1), dp(s1), dp(v1), n1, ip(q1), np_(r1),
                       int(g2['type']), dp(p2), dp(m2), dp(s2), dp(v2), n2, ip(q2), np_(r2),
                       ct.c_double(margin), ct.c_double(gap), int(boxbox == 'primitive') | (2 if convex in ('mpr', 'mpr64') else 0) | (4 if convex == 'mpr64' else 0),
                       ct.c_double(tolerance), int(iterations), int(epa_iterations), dp(op), dp(on), dp(od), maxout)
    if n < 0:
        raise ValueError('geom pair not supported by the oracle narrowphase')
    return op[:3 * n].reshape(n, 3), on[:3 * n].reshape(n, 3), od[:n]
