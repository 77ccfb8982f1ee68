"""Correctness oracle -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker.  The product (the
``hip`` plugin under ``chomik-grad_amd/``) never imports it.

``numpy_plugin`` restates the reference's NumPy ``cpu`` plugin
(chomikgrad/lazy.py:502-636) and registers it as ``cpu``.
"""

from .numpy_plugin import NumpyCompiler, NumpyDeviceAdapter, NumpyProgram, install

__all__ = ["NumpyCompiler", "NumpyDeviceAdapter", "NumpyProgram", "install"]
