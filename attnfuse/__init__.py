"""Drop-in import name: ``import attnfuse as af`` resolves to
``attentionfuse_amd`` and every ``attnfuse.<sub.module>`` path of the
reference package (dsl, ir, compiler, runtime, rope_utils, integrations)
names the same module object, so isinstance checks and monkeypatching work
across both names."""
import importlib
import sys

import attentionfuse_amd as _impl

_SUBMODULES = [
    "dsl", "dsl.api", "dsl.tracer",
    "ir", "ir.high_level", "ir.spec", "ir.printer",
    "compiler", "compiler.fusion", "compiler.lowering", "compiler.tiling",
    "runtime", "runtime._native", "runtime.dispatch", "runtime.kernel_cache",
    "runtime.flash_decode", "runtime.backward", "runtime.block_mask",
    "runtime.autograd",
    "rope_utils",
]

for _name in _SUBMODULES:
    sys.modules[f"{__name__}.{_name}"] = importlib.import_module(
        f"attentionfuse_amd.{_name}")

# The reference keeps the lowered record in attnfuse.ir.tiled.
sys.modules[f"{__name__}.ir.tiled"] = sys.modules["attentionfuse_amd.ir.spec"]

from attentionfuse_amd import *  # noqa: E402,F401,F403
from attentionfuse_amd import __all__, __version__  # noqa: E402,F401

dsl = _impl.dsl
ir = _impl.ir
compiler = _impl.compiler
runtime = _impl.runtime
rope_utils = _impl.rope_utils
