"""``dsl_splat.splatting.cameras`` is ``dsl_splat_amd.splatting.cameras`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.splatting.cameras")
