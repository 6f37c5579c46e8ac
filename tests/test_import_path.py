"""The reference's import path (dsl_splat.gs3d ...) resolves to dsl_splat_amd's
modules when dsl_splat_amd/compat is on sys.path (checked in a fresh
interpreter, so nothing here is imported from the test process)."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import sys
import dsl_splat
from dsl_splat import gs3d
from dsl_splat.gs3d import RasterizationResult, ops, rasterize
from dsl_splat.gs3d.gsplat import rasterization
from dsl_splat.gs3d.ops import bin_and_sort, prepare_gaussians, rasterize_to_pixels, spherical_harmonics
from dsl_splat.cameras import PinholeCamera
from dsl_splat.statistics import MaskedContributionCount, WeightedContributionSum
from dsl_splat.primitives.tiling import sort_tile_pairs
import dsl_splat.training, dsl_splat.inputs, dsl_splat.primitives.spherical_harmonics
import dsl_splat_amd.gs3d, dsl_splat_amd.gs3d.gsplat, dsl_splat_amd.cameras, dsl_splat_amd.statistics
import dsl_splat_amd.primitives.tiling
assert rasterize is dsl_splat_amd.gs3d.rasterize
assert RasterizationResult is dsl_splat_amd.gs3d.RasterizationResult
assert ops is dsl_splat_amd.gs3d.ops and gs3d.ops is ops and dsl_splat.gs3d.ops is ops
assert rasterization is dsl_splat_amd.gs3d.gsplat.rasterization
assert PinholeCamera is dsl_splat_amd.cameras.PinholeCamera is dsl_splat.PinholeCamera
assert MaskedContributionCount is dsl_splat_amd.statistics.MaskedContributionCount
assert sort_tile_pairs is dsl_splat_amd.primitives.tiling.sort_tile_pairs
import dsl_splat.gs3d.render, dsl_splat.gs3d.projection, dsl_splat.gs3d.binning, dsl_splat.gs3d.cameras
import dsl_splat.gs3d.api, dsl_splat.gs3d.autograd
import dsl_splat.splatting.binning, dsl_splat.splatting.cameras, dsl_splat.splatting.geometry
import dsl_splat.runtime.gradients
from dsl_splat.gs3d.binning import bin_and_sort as gs3d_bin_and_sort
from dsl_splat.splatting.geometry import ProjectedGaussians
from dsl_splat.runtime.gradients import AbsGradientTarget
import dsl_splat_amd.gs3d.binning, dsl_splat_amd.splatting.geometry, dsl_splat_amd.runtime.gradients
assert gs3d_bin_and_sort is dsl_splat_amd.gs3d.binning.bin_and_sort
assert ProjectedGaussians is dsl_splat_amd.splatting.geometry.ProjectedGaussians
assert AbsGradientTarget is dsl_splat_amd.runtime.gradients.AbsGradientTarget
for name in ("gs3d.gsplat", "gs3d.ops", "cameras", "statistics", "training", "inputs", "primitives.tiling",
             "primitives.spherical_harmonics", "gs3d.api", "gs3d.autograd", "gs3d.binning", "gs3d.cameras",
             "gs3d.projection", "gs3d.render", "splatting.binning", "splatting.cameras", "splatting.geometry",
             "runtime.gradients"):
    assert sys.modules["dsl_splat." + name] is sys.modules["dsl_splat_amd." + name], name
print("ok")
"""


def test_reference_import_path_resolves_to_this_build():
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([os.path.join(ROOT, "dsl_splat_amd", "compat"), ROOT]))
    run = subprocess.run([sys.executable, "-c", SCRIPT], cwd="/", env=env, capture_output=True, text=True)
    assert run.returncode == 0, run.stderr[-3000:]
    assert run.stdout.strip() == "ok"
