"""Parity at the benchmark workloads' full sizes.

Each workload is built at its stated size (synthetic.make_scene) and run
forward + backward through gs3d.rasterize on the GPU, then through the
oracle pipeline on all host cores:

  1. 10,000 Gaussians, 256x256, RGB features, one camera (also as degree-0 SH)
  2. 500,000 Gaussians, 1280x720, SH degree 3, absgrad
  3. 3,000,000 Gaussians in 64 clusters, SH degree 3, four 1920x1080 cameras
  4. 1,000,000 Gaussians, 1600x1200, 32 feature channels + camera-z channel
  5. 2,000,000 Gaussians (5% large), 1920x1080, SH3, pose gradients, absgrad

Bit-exact: images (every channel and alpha), radii, tile counts, means2d,
conics, opacities, and the binning -- every tile's Gaussian ids, the tile
ranges and the reference's 64-bit sort keys -- against the oracle's scan,
emission and stable radix sort.  Gradients: every entry within
rtol 1e-4 / atol 1e-5 of the oracle or its float32 error bound.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from dsl_splat_amd import synthetic
from dsl_splat_amd.gs3d import projection as gproj
from dsl_splat_amd.splatting import binning, cameras
from test_gpu_rasterize import run_scene

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]
DEV = "cuda"
THREADS = len(os.sched_getaffinity(0))


def _check_binning(scene, ref):
    """The product's binning of the same projected rows against the oracle's
    scan + emission + stable sort: ids, ranges and 64-bit keys."""
    with_centers = scene.sh_degree is not None and scene.sh_degree > 0
    full, _, centers, _ = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height, with_centers)
    st = gproj.project_views(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, full,
                             scene.Ks, scene.width, scene.height, 0.2, float("inf"), 0.0, normalize_quats=True)
    bins = binning.bin_and_sort(st.centers, st.radii, st.tile_counts, st.depths, scene.width, scene.height,
                                with_keys=True)
    count = int(ref["total"])
    print(f"  binning: {count} tile pairs", flush=True)
    assert bins["point_list"].numel() == count
    np.testing.assert_array_equal(bins["ranges"].cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(bins["point_list"].cpu().numpy(), ref["sorted_vals"])
    np.testing.assert_array_equal(bins["point_list_keys"].cpu().numpy().view(np.uint64),
                                  ref["sorted_keys"].view(np.uint64))


def _run(scene):
    print(f"workload {scene.name}: n={len(scene.means)} views={scene.viewmats.shape[0]} "
          f"{scene.width}x{scene.height}, oracle on {THREADS} threads", flush=True)
    image, meta, ref = run_scene(scene, oracle_threads=THREADS)
    _check_binning(scene, ref)
    del ref
    oracle.set_threads(1)


def test_workload_1_rgb_256():
    _run(synthetic.make_scene("small", seed=0).to(DEV))


def test_workload_1_sh0_256():
    scene = synthetic.make_scene("small", seed=0)
    # The same colours as degree-0 SH: colour = max(0.28209479 c + 0.5, 0).
    scene.sh_coeffs = ((scene.features - 0.5) / 0.28209479)[:, None, :].contiguous()
    scene.sh_degree, scene.features = 0, None
    _run(scene.to(DEV))


def test_workload_2_sh3_720p_absgrad():
    _run(synthetic.make_scene("sh3_720p", seed=0).to(DEV))


def test_workload_3_sh3_1080p_4_cameras():
    _run(synthetic.make_scene("sh3_1080p_4view", seed=0).to(DEV))


def test_workload_4_feat32_depth_1200p():
    _run(synthetic.make_scene("feat32", seed=0).to(DEV))


def test_workload_5_pose_fanout_1080p():
    _run(synthetic.make_scene("pose_fanout", seed=0).to(DEV))
