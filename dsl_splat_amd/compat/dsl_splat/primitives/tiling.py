"""``dsl_splat.primitives.tiling`` is ``dsl_splat_amd.primitives.tiling`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.primitives.tiling")
