"""``tilegen``: the import path TileGen's own scripts and tests use.

``from tilegen.codegen import Config, generate``, ``from tilegen import passes``,
``from tilegen.autotune import BASELINE, tune, write_outputs`` and the like
resolve to this build's modules in ``tilegen_amd``: ``tilegen.<m>`` is the very
module object ``tilegen_amd.<m>`` (the same classes, caches and loaded
libraries, whichever name a caller imports), so callers written against the
reference package run unchanged on the HIP backend.

The modules are the reference package's eight (env, matrices, dsl, ir, passes,
codegen, verify, autotune).  Names that exist only for CUDA in the reference
(``verify.cuda_arch``, ``codegen.emit_cuda``, the CUDA text checks of
``verify``) have HIP counterparts here under HIP names (``verify.hip_arch``,
``codegen.emit_hip``); there is no CUDA path to alias them to.
"""

import importlib
import sys

import tilegen_amd as _impl

MODULES = ("env", "matrices", "dsl", "ir", "passes", "codegen", "verify", "autotune")

for _name in MODULES:
    _mod = importlib.import_module("tilegen_amd." + _name)
    sys.modules[__name__ + "." + _name] = _mod
    globals()[_name] = _mod
del _name, _mod

__version__ = _impl.__version__

__all__ = ["__version__"] + list(MODULES)
