"""Host side of the MI355X resident continuous decode step.

- ``rstr.hip``: ctypes binding of ``librstr_hip.so`` (the C ABI in include/rstr_hip.h).
- ``rstr.configs``: model descriptors of the benchmark shapes.
"""
