"""The reference package's import path for the 3DGS rasterizer.

With this directory (``dsl_splat_amd/compat``) ahead of the reference on
``sys.path``, code written against ``dsl_splat.gs3d`` (``rasterize``,
``RasterizationResult``, ``ops``, ``gsplat.rasterization`` and the modules
``api``, ``autograd``, ``binning``, ``cameras``, ``projection``, ``render``),
``dsl_splat.splatting.{binning,cameras,geometry}``, ``dsl_splat.cameras``,
``dsl_splat.statistics``, ``dsl_splat.training``, ``dsl_splat.inputs``,
``dsl_splat.runtime.gradients`` and ``dsl_splat.primitives.tiling`` /
``.spherical_harmonics`` runs unchanged on the HIP build: every module here is
the ``dsl_splat_amd`` module of the same name (one object, not a copy).  The
reference's Warp kernel modules (``gs3d/frame.py``, ``*/math.py``,
``*/metadata.py``, ``*/camera_kernels.py``, ``splatting/intersections.py``,
``runtime/dispatch.py``) have no Python counterpart: the HIP library does
their work behind the same entry points.  The reference's other methods (its
root exports, aaa, geer, pgsr, rade, strategy) are not part of dsl_splat_amd.
"""

import importlib

from dsl_splat_amd.cameras import PinholeCamera

__all__ = ["PinholeCamera", "gs3d"]


def __getattr__(name):
    if name == "gs3d":
        return importlib.import_module(f"{__name__}.gs3d")
    raise AttributeError(name)
