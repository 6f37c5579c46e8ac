"""MI355X-native original-3DGS rasterizer with the dsl_splat gs3d interface.

Use ``dsl_splat_amd.gs3d.rasterize`` (method API) or
``dsl_splat_amd.gs3d.gsplat.rasterization`` (gsplat signature).  Unlike the
reference package root, importing this package loads no other method.
"""

import importlib

from .cameras import PinholeCamera

__all__ = ["PinholeCamera", "gs3d"]


def __getattr__(name):
    if name == "gs3d":
        return importlib.import_module(f"{__name__}.gs3d")
    raise AttributeError(name)
