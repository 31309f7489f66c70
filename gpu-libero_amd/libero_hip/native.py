"""ctypes binding of libmx_physics.so and the device-resident model / batch buffers.

The reference binds one ctypes ``Structure`` of pointers and ints per leaf library and checks
``arguments_bytes``/``arch`` at load (``gpu/host/runtime/dynamics/mjwarp_motion.py:20-37``,
``gpu/host/backends/cuda_fp32/controller.py:92-99``).  This module does the same for the single
world-local library.  PyTorch-ROCm owns every device buffer (model arenas and per-world arrays);
the library receives raw pointers and never allocates.  There is no CPU fallback: a missing or
mismatched library raises.
"""
from __future__ import annotations

import ctypes as ct
from pathlib import Path

import numpy as np

from . import layout

PACKAGE = Path(__file__).resolve().parent.parent
LIBRARY = PACKAGE / 'libmx_physics.so'

MxModel = layout.make_struct('MxModel', ct.c_float, ct.c_float, 'model')
MxData = layout.make_struct('MxData', ct.c_float, ct.c_float, 'data')

FLAG_POLICY_FIRST, FLAG_NO_CONTROL, FLAG_NO_INTEGRATE, FLAG_BOOTSTRAP, FLAG_WORKSPACE, FLAG_LDS = 1, 2, 4, 8, 16, 32
FLAG_FP64 = 64   # the FP64 route (physics in double, working set in LDS)

EXPORTS = ['mx_abi_version', 'mx_model_bytes', 'mx_data_bytes', 'mx_arch', 'mx_source_id',
           'mx_field_count', 'mx_field_name', 'mx_check', 'mx_lds_bytes', 'mx_lds_bytes_fp64', 'mx_workspace_bytes',
           'mx_control_step',
           'mx_control_step_noalloc', 'mx_forward', 'mx_control_step_observed', 'mx_observe', 'mx_observe_reset',
           'mx_obs_plan_bytes', 'mx_osc', 'mx_error_string']


class MxObsPlan(ct.Structure):
    """ctypes mirror of MxObsPlan (include/mx_physics.h): the plan's metadata and per-world state."""
    _fields_ = ([('nspec', ct.c_int32), ('width', ct.c_int32)]
                + [(n, ct.POINTER(ct.c_int32)) for n in ('op', 'offset', 'size', 'index_offset', 'indices', 'dep0',
                                                         'dep1', 'dep2', 'presence', 'enabled')]
                + [('period', ct.POINTER(ct.c_float))]
                + [(n, ct.POINTER(ct.c_float)) for n in ('cache', 'observed', 'sidequat', 'elapsed')]
                + [(n, ct.POINTER(ct.c_int32)) for n in ('sampled', 'present', 'events')])

# mx_control_step_noalloc's fixed device scratch (MX_SCRATCH_BYTES) and its refusal code
SCRATCH_BYTES = 64 << 20
ERR_SCRATCH = -4

_LIB = None


def load(path=None):
    """Load and ABI-check the library (no GPU call is made)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIBRARY
    if not p.exists():
        raise ImportError('libmx_physics.so is not built (%s); run gpu-libero_amd/build.py' % p)
    lib = ct.CDLL(str(p))
    lib.mx_abi_version.restype = ct.c_int
    lib.mx_model_bytes.restype = ct.c_size_t
    lib.mx_data_bytes.restype = ct.c_size_t
    lib.mx_arch.restype = ct.c_int
    lib.mx_source_id.restype = ct.c_char_p
    lib.mx_field_count.restype = ct.c_int
    lib.mx_field_count.argtypes = [ct.c_int]
    lib.mx_field_name.restype = ct.c_char_p
    lib.mx_field_name.argtypes = [ct.c_int, ct.c_int]
    lib.mx_check.argtypes = [ct.c_void_p, ct.c_void_p]
    lib.mx_lds_bytes.argtypes = [ct.c_void_p]
    lib.mx_lds_bytes_fp64.argtypes = [ct.c_void_p]
    lib.mx_workspace_bytes.restype = ct.c_size_t
    lib.mx_workspace_bytes.argtypes = [ct.c_void_p]
    lib.mx_control_step.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p]
    lib.mx_control_step_noalloc.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p]
    lib.mx_control_step_observed.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p]
    lib.mx_observe.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_float, ct.c_int, ct.c_void_p]
    lib.mx_observe_reset.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p]
    lib.mx_osc.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_void_p]
    lib.mx_forward.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_void_p]
    lib.mx_error_string.restype = ct.c_char_p
    lib.mx_error_string.argtypes = [ct.c_int]
    if lib.mx_abi_version() != layout.ABI_VERSION:
        raise ImportError('libmx_physics ABI version %d != %d' % (lib.mx_abi_version(), layout.ABI_VERSION))
    lib.mx_obs_plan_bytes.restype = ct.c_size_t
    if (lib.mx_model_bytes() != ct.sizeof(MxModel) or lib.mx_data_bytes() != ct.sizeof(MxData)
            or lib.mx_obs_plan_bytes() != ct.sizeof(MxObsPlan)):
        raise ImportError('libmx_physics struct sizes differ from the Python mirror')
    if lib.mx_arch() != 950:
        raise ImportError('libmx_physics was not built for gfx950')
    layout.check_field_tables(lib.mx_field_count, lib.mx_field_name, 'libmx_physics')
    if path is None:
        _LIB = lib
    return lib


def check(rc, what):
    if rc != 0:
        msg = load().mx_error_string(rc).decode()
        raise RuntimeError('%s failed: %s (%d)' % (what, msg, rc))


class DeviceModel:
    """Model arrays uploaded to one float arena and one int arena on the device."""

    def __init__(self, model, device='cuda:0'):
        import torch
        self.model = model
        real, ints = layout.model_arrays(model)
        farena, foff = layout.pack_arena(real, np.float32)
        iarena, ioff = layout.pack_arena(ints, np.int32)
        self.farena = torch.from_numpy(farena).to(device)
        self.iarena = torch.from_numpy(iarena).to(device)
        s = MxModel()
        for k, v in layout.model_scalars(model).items():
            setattr(s, k, v)
        fbase, ibase = self.farena.data_ptr(), self.iarena.data_ptr()
        for name in layout.MODEL_REAL_ARRAYS:
            setattr(s, name, ct.cast(ct.c_void_p(fbase + 4 * foff[name]), ct.POINTER(ct.c_float)))
        for name in layout.MODEL_INT_ARRAYS:
            setattr(s, name, ct.cast(ct.c_void_p(ibase + 4 * ioff[name]), ct.POINTER(ct.c_int32)))
        self.struct = s

    def lds_bytes(self):
        return load().mx_lds_bytes(ct.byref(self.struct))

    def lds_bytes_fp64(self):
        return load().mx_lds_bytes_fp64(ct.byref(self.struct))


class DeviceData:
    """Per-world arrays (world-major) as torch tensors, and the MxData pointer struct."""

    def __init__(self, dmodel, nworld, device='cuda:0', workspace=None, validate=True):
        """``workspace``: None allocates the per-world workspace slabs for models with constraint rows
        (the faster route) and for models beyond the LDS budget; True always; False never (the LDS
        route, for models that fit, or ``control_step_noalloc`` with ``validate=False`` for models
        beyond LDS, whose slabs come from the library's fixed scratch)."""
        import torch
        self.dmodel = dmodel
        m = dmodel.model
        self.nworld = nworld
        if workspace is None:
            workspace = m.njmax > 0 or dmodel.lds_bytes() > layout.LDS_BUDGET
        ws = load().mx_workspace_bytes(ct.byref(dmodel.struct)) // 8 if workspace else 0
        widths = layout.data_widths(m, ws)
        self.arrays = {}
        s = MxData()
        s.nworld = nworld
        s.workspace_doubles = ws
        s.workspace_total = (nworld + 1) * ws if ws else 0
        for name in layout.DATA_REAL_ARRAYS:
            t = torch.zeros((nworld, max(widths[name], 1)), dtype=torch.float32, device=device)
            self.arrays[name] = t
            setattr(s, name, ct.cast(ct.c_void_p(t.data_ptr()), ct.POINTER(ct.c_float)))
        for name in layout.DATA_F64_ARRAYS:
            rows = nworld + 1 if name == 'workspace' and ws else nworld   # slab 0: the model image
            t = torch.zeros((rows, max(widths[name], 1)), dtype=torch.float64, device=device)
            self.arrays[name] = t
            setattr(s, name, ct.cast(ct.c_void_p(t.data_ptr()), ct.POINTER(ct.c_double)))
        for name in layout.DATA_INT_ARRAYS:
            t = torch.zeros((nworld, max(widths[name], 1)), dtype=torch.int32, device=device)
            self.arrays[name] = t
            setattr(s, name, ct.cast(ct.c_void_p(t.data_ptr()), ct.POINTER(ct.c_int32)))
        self.struct = s
        # every world starts with the model's action ranges (read when m.osc_action_scaled)
        self.arrays['osc_action_scale'].copy_(torch.from_numpy(m.osc_action_scale).expand(nworld, -1))
        if validate:
            check(load().mx_check(ct.byref(dmodel.struct), ct.byref(s)), 'mx_check')

    def __getitem__(self, name):
        return self.arrays[name]

    def _stream(self, stream):
        import torch
        if stream is None:
            stream = torch.cuda.current_stream()
        return ct.c_void_p(stream.cuda_stream)

    def control_step(self, substeps, flags=FLAG_POLICY_FIRST, stream=None):
        rc = load().mx_control_step(ct.byref(self.dmodel.struct), ct.byref(self.struct), substeps, flags,
                                    self._stream(stream))
        check(rc, 'mx_control_step')

    def control_step_noalloc(self, substeps, flags=FLAG_POLICY_FIRST, stream=None):
        """mx_control_step with the library's fixed device scratch as the workspace (no allocation)."""
        rc = load().mx_control_step_noalloc(ct.byref(self.dmodel.struct), ct.byref(self.struct), substeps, flags,
                                            self._stream(stream))
        check(rc, 'mx_control_step_noalloc')

    def osc(self, flags=0, stream=None):
        """mx_osc: the FP64 controller alone from the published controller inputs."""
        rc = load().mx_osc(ct.byref(self.dmodel.struct), ct.byref(self.struct), flags, self._stream(stream))
        check(rc, 'mx_osc')

    def forward(self, mask=None, flags=0, stream=None):
        ptr = None if mask is None else ct.c_void_p(mask.data_ptr())
        rc = load().mx_forward(ct.byref(self.dmodel.struct), ct.byref(self.struct), ptr, flags,
                               self._stream(stream))
        check(rc, 'mx_forward')
