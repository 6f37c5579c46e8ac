"""``dsl_splat.runtime.gradients`` is ``dsl_splat_amd.runtime.gradients`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.runtime.gradients")
