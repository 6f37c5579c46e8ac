"""``dsl_splat.training`` is ``dsl_splat_amd.training`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.training")
