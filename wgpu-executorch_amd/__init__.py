"""wgpu-executorch_amd: the MI355X (gfx950) hot path of wgpu-executorch.

The kernels live in ``csrc/`` and are reached only through the C-ABI library
``libwgx.so`` (``include/wgx.h``).  ``wgx`` is the Python binding of that ABI,
``js/`` the Node binding with the reference's TypeScript-facing API,
``inputs`` the seeded synthetic inputs, ``program`` the program.json runner.

The directory name is not a Python identifier; load it with ``load()`` below
or ``importlib`` (tests/conftest.py, bench.py and __graft_entry__.py do).
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))

from . import inputs, wgx  # noqa: E402,F401

__all__ = ["wgx", "inputs", "HERE"]
