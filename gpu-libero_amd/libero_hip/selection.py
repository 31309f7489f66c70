"""Engine routing with the new ``hip_mi355x`` route.

Mirrors ``resolve_engine`` (``gpu/host/backends/selection.py:5-17``): same argument meaning and
ValueError behaviour for bad choices, with ``'hip_mi355x'`` added as the FP32 route of this
backend (``'auto'`` at FP32 resolves to it).  The reference's other engines are not part of this
build and are rejected with a ValueError naming them.
"""

ENGINES = ('auto', 'native', 'mjwarp', 'cuda_fp32', 'hip_mi355x')


def resolve_engine(engine='auto', precision=None):
    if engine not in ENGINES:
        raise ValueError('physics_engine must be auto, native, mjwarp, cuda_fp32 or hip_mi355x')
    if precision is not None and precision not in ('fp32', 'float32', 'fp64', 'float64'):
        raise ValueError('precision must be fp32 or fp64')
    bits = 32 if precision is None or precision in ('fp32', 'float32') else 64
    if engine == 'auto':
        engine = 'hip_mi355x' if bits == 32 else 'native'
    if engine == 'hip_mi355x' and bits == 64:
        raise ValueError('hip_mi355x runs FP32 physics with an FP64 controller; FP64 physics is not provided')
    if engine != 'hip_mi355x':
        raise ValueError('physics_engine=%r is a reference engine that this MI355X build does not provide' % engine)
    return engine
