"""``dsl_splat.inputs`` is ``dsl_splat_amd.inputs`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.inputs")
