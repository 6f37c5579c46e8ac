"""The reference's limits, not narrower ones: any number of cameras with pose
gradients (the reference launches its projection VJP per view,
gs3d/api.py:132-189), and an int32 pair capacity per view rather than per
frame (primitives/tiling.py:57-64, splatting/binning.py:88-89).  Each case
runs forward + backward and is compared with the oracle."""

import math

import numpy as np
import pytest
import torch

from dsl_splat_amd import gs3d, synthetic
from dsl_splat_amd.gs3d import projection as gproj
from dsl_splat_amd.splatting import binning
from test_gpu_rasterize import run_scene

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ring_scene(cameras, n=2500, width=112, height=72, seed=81):
    scene = synthetic.make_scene("sh3_720p", n=n, width=width, height=height, seed=seed)
    scene.viewmats = torch.stack([
        synthetic.look_at((4.0 * math.sin(2 * math.pi * c / cameras), 0.3 * math.cos(c),
                           -4.0 * math.cos(2 * math.pi * c / cameras))) for c in range(cameras)])
    scene.Ks = scene.Ks.repeat(cameras, 1, 1)
    g = torch.Generator().manual_seed(seed)
    scene.loss_weights = torch.randn((cameras, height, width, 4), generator=g)
    scene.pose_grad = True
    return scene.to(DEV)


def test_camera_gradients_for_more_cameras_than_one_launch_group():
    cameras = gproj.CAMERA_GRADIENT_GROUP + 2
    print(f"pose gradients, {cameras} cameras", flush=True)
    run_scene(_ring_scene(cameras))


def test_pair_capacity_is_per_view(monkeypatch):
    # Lower the per-launch pair capacity below the frame's total so that the
    # cameras are binned and blended in groups; the result must not change.
    scene = _ring_scene(5, n=3000, seed=83)
    args = (scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, scene.width,
            scene.height)
    whole = gs3d.rasterize(*args, sh_coeffs=scene.sh_coeffs)
    per_view = whole.meta["tiles_per_gauss"].sum(dim=-1).tolist()
    limit = 2 * max(per_view) + 1  # two cameras per group, not three
    monkeypatch.setattr(binning, "PAIR_LIMIT", limit)
    groups = binning.view_groups(per_view)
    print(f"pairs per view {per_view}, limit {limit}, groups {groups}", flush=True)
    assert 1 < len(groups) < len(per_view)
    split = gs3d.rasterize(*args, sh_coeffs=scene.sh_coeffs)
    assert torch.equal(split.features, whole.features) and torch.equal(split.alpha, whole.alpha)
    run_scene(scene)
    # One view above the capacity is the reference's overflow too.
    monkeypatch.setattr(binning, "PAIR_LIMIT", max(per_view) - 1)
    with pytest.raises(OverflowError):
        gs3d.rasterize(*args, sh_coeffs=scene.sh_coeffs)
