"""Package directory of the MI355X backend: ``csrc/`` (HIP kernels + C ABI), ``libero_hip/``
(Python host side), ``build.py`` (hipcc build of ``libmx_physics.so``)."""
