"""Engine routing with the new ``hip_mi355x`` route.

Mirrors ``resolve_engine`` (``gpu/host/backends/selection.py:5-17``): same argument meaning and
ValueError behaviour for bad choices, with ``'hip_mi355x'`` added as this backend's engine.  It
runs at both precisions: FP32 physics (the reference's ``cuda_fp32`` role; ``'auto'`` at FP32
resolves to it) and the FP64 route (physics in double with the working set in LDS; ``'auto'`` at
FP64 resolves to it where the reference picks its FP64 ``'native'`` engine).  The reference's other
engines are not part of this build and are rejected with a ValueError naming them.
"""

ENGINES = ('auto', 'native', 'mjwarp', 'cuda_fp32', 'hip_mi355x')


def precision_bits(precision=None):
    """32 or 64 for a precision argument (None: FP32); ValueError as the reference for others."""
    if precision is not None and precision not in ('fp32', 'float32', 'fp64', 'float64'):
        raise ValueError('precision must be fp32 or fp64')
    return 32 if precision is None or precision in ('fp32', 'float32') else 64


def resolve_engine(engine='auto', precision=None):
    if engine not in ENGINES:
        raise ValueError('physics_engine must be auto, native, mjwarp, cuda_fp32 or hip_mi355x')
    precision_bits(precision)
    if engine == 'auto':
        engine = 'hip_mi355x'
    if engine != 'hip_mi355x':
        raise ValueError('physics_engine=%r is a reference engine that this MI355X build does not provide' % engine)
    return engine
