"""``dsl_splat.primitives.spherical_harmonics`` is ``dsl_splat_amd.primitives.spherical_harmonics`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.primitives.spherical_harmonics")
