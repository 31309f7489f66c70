"""Host side of the FP64 route (no GPU): engine selection at both precisions, the route's launch
flag, and its LDS sizing (every physics value in double, the model image and the integer arrays
unchanged): larger than the FP32 route's, at most twice it, within the 160 KiB of a workgroup for
C1, C2 and C3 and beyond it for C4 and C5 (which then have no FP64 route)."""
import ctypes as ct

import pytest

from libero_hip import layout, native
from libero_hip import scene as S
from libero_hip.model import Model
from libero_hip.selection import precision_bits, resolve_engine


def test_engine_selection_admits_fp64():
    assert resolve_engine('auto', 'fp64') == 'hip_mi355x'
    assert resolve_engine('hip_mi355x', 'float64') == 'hip_mi355x'
    assert resolve_engine() == 'hip_mi355x'
    assert precision_bits('fp64') == 64 and precision_bits(None) == 32
    with pytest.raises(ValueError, match='precision'):
        resolve_engine('hip_mi355x', 'fp16')
    for engine in ('native', 'mjwarp', 'cuda_fp32'):
        with pytest.raises(ValueError, match='does not provide'):
            resolve_engine(engine, 'fp64')
    with pytest.raises(ValueError, match='physics_engine'):
        resolve_engine('warp')


def test_fp64_flag_is_distinct():
    flags = [native.FLAG_POLICY_FIRST, native.FLAG_NO_CONTROL, native.FLAG_NO_INTEGRATE, native.FLAG_BOOTSTRAP,
             native.FLAG_WORKSPACE, native.FLAG_LDS, native.FLAG_FP64]
    assert native.FLAG_FP64 == 64 and len(set(flags)) == len(flags)


@pytest.mark.parametrize('config,fits', [('c1', True), ('c2', True), ('c3', True), ('c4', False), ('c5', False)])
def test_fp64_lds_sizes(config, fits):
    m = Model(S.make_scene(config, 2, seed=0))
    s = native.MxModel()
    for k, v in layout.model_scalars(m).items():
        setattr(s, k, v)
    lib = native.load()
    b32, b64 = lib.mx_lds_bytes(ct.byref(s)), lib.mx_lds_bytes_fp64(ct.byref(s))
    assert b32 < b64 < 2 * b32
    assert (b64 <= layout.LDS_BUDGET) == fits
    assert lib.mx_lds_bytes_fp64(None) == -1
