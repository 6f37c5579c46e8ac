"""``dsl_splat.gs3d.projection`` is ``dsl_splat_amd.gs3d.projection`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.gs3d.projection")
