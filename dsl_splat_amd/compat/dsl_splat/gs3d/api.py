"""``dsl_splat.gs3d.api`` is ``dsl_splat_amd.gs3d.api`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.gs3d.api")
