"""``dsl_splat.splatting.binning`` is ``dsl_splat_amd.splatting.binning`` (the same module object)."""

import importlib
import sys

sys.modules[__name__] = importlib.import_module("dsl_splat_amd.splatting.binning")
