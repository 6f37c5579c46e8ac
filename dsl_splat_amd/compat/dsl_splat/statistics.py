"""``dsl_splat.statistics`` is ``dsl_splat_amd.statistics`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.statistics")
