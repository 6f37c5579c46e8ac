"""``dsl_splat.gs3d.render`` is ``dsl_splat_amd.gs3d.render`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.gs3d.render")
