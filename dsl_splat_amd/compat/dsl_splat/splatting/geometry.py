"""``dsl_splat.splatting.geometry`` is ``dsl_splat_amd.splatting.geometry`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.splatting.geometry")
