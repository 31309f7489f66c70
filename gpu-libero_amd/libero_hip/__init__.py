"""MI355X-native batched physics backend for GPU-LIBERO's per-world control step.

Route: ``physics_engine='hip_mi355x'`` (see :mod:`libero_hip.selection`).  The façade is
:class:`libero_hip.environment.HipBatchEnv`; the device code is ``libmx_physics.so`` (C ABI in
``include/mx_physics.h``), bound by :mod:`libero_hip.native`.
"""
from .selection import resolve_engine  # noqa: F401

__all__ = ['resolve_engine']
