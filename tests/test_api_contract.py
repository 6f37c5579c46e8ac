"""Host-side contract of the public entry points (no GPU needed): the same
validation errors and exception types as the reference's gs3d.rasterize
(gs3d/api.py:86-102), gsplat adapter (gs3d/gsplat.py:15-84), camera options
(cameras.py:30-41), inputs (inputs.py:164-243) and statistics requests
(statistics.py:72-128)."""

import math

import pytest
import torch

from dsl_splat_amd import gs3d
from dsl_splat_amd.cameras import validate_camera_options
from dsl_splat_amd.gs3d import gsplat
from dsl_splat_amd.statistics import MaskedContributionCount, WeightedContributionSum, prepare_statistics


def _cpu_scene(n=8):
    return dict(
        means=torch.zeros(n, 3), quats=torch.zeros(n, 4), scales=torch.ones(n, 3), opacities=torch.ones(n),
        viewmats=torch.eye(4)[None], Ks=torch.eye(3)[None],
    )


def test_rasterize_option_errors():
    s = _cpu_scene()
    args = (s["means"], s["quats"], s["scales"], s["opacities"], s["viewmats"], s["Ks"], 32, 32)
    with pytest.raises(ValueError, match="tile_mode"):
        gs3d.rasterize(*args, features=torch.zeros(8, 3), tile_mode="box")
    with pytest.raises(ValueError, match="width and height"):
        gs3d.rasterize(*args[:6], 0, 32, features=torch.zeros(8, 3))
    with pytest.raises(ValueError, match="near_plane"):
        gs3d.rasterize(*args, features=torch.zeros(8, 3), near_plane=-1.0)
    with pytest.raises(ValueError, match="radius_clip"):
        gs3d.rasterize(*args, features=torch.zeros(8, 3), radius_clip=math.inf)
    with pytest.raises(ValueError, match="exactly one of features or sh_coeffs"):
        gs3d.rasterize(*args)
    with pytest.raises(ValueError, match="exactly one of features or sh_coeffs"):
        gs3d.rasterize(*args, features=torch.zeros(8, 3), sh_coeffs=torch.zeros(8, 16, 3))
    with pytest.raises(ValueError, match="sh_degree requires sh_coeffs"):
        gs3d.rasterize(*args, features=torch.zeros(8, 3), sh_degree=2)
    with pytest.raises(ValueError, match="sh_degree must be an integer"):
        gs3d.rasterize(*args, sh_coeffs=torch.zeros(8, 16, 3), sh_degree=4)
    with pytest.raises(ValueError, match="sh_coeffs must have shape"):
        gs3d.rasterize(*args, sh_coeffs=torch.zeros(8, 3))
    # Host tensors are rejected before anything reaches a device.
    with pytest.raises(ValueError, match="means must be a CUDA float32 tensor"):
        gs3d.rasterize(*args, features=torch.zeros(8, 3))


def test_camera_option_validation():
    validate_camera_options(10, 10, 0.1, math.inf, 0.0)
    for bad in ((0, 10, 0.1, 1.0, 0.0), (10, True, 0.1, 1.0, 0.0), (10, 10, 0.0, 1.0, 0.0),
                (10, 10, 1.0, 1.0, 0.0), (10, 10, 0.1, math.nan, 0.0), (10, 10, 0.1, 1.0, -1.0)):
        with pytest.raises(ValueError):
            validate_camera_options(*bad)


@pytest.mark.parametrize("kwargs,exc", [
    (dict(sparse_grad=True), NotImplementedError), (dict(distributed=True), NotImplementedError),
    (dict(segmented=True), NotImplementedError), (dict(with_ut=True), NotImplementedError),
    (dict(covars=torch.zeros(1)), NotImplementedError), (dict(radial_coeffs=torch.zeros(1)), NotImplementedError),
    (dict(extra_signals_sh_degree=1), NotImplementedError), (dict(rolling_shutter="ROLLING"), NotImplementedError),
    (dict(camera_model="fisheye"), NotImplementedError), (dict(with_eval3d=True), NotImplementedError),
    (dict(eps2d=0.1), NotImplementedError), (dict(tile_size=8), NotImplementedError),
    (dict(render_mode="RGB+D"), NotImplementedError), (dict(rasterize_mode="antialiased"), NotImplementedError),
    (dict(channel_chunk=0), ValueError), (dict(near_plane=0.0), ValueError), (dict(sh_degree=5), ValueError),
])
def test_gsplat_adapter_rejects_unsupported_options(kwargs, exc):
    s = _cpu_scene()
    with pytest.raises(exc):
        gsplat.rasterization(s["means"], s["quats"], s["scales"], s["opacities"], torch.zeros(8, 3), s["viewmats"],
                             s["Ks"], 32, 32, **kwargs)


def test_statistics_request_validation():
    H, W = 4, 5
    mask = torch.zeros((H, W), dtype=torch.bool)
    weights = torch.ones((H, W))
    prepared, outputs = prepare_statistics(
        [MaskedContributionCount("hits", mask), WeightedContributionSum("score", weights)],
        batch_dims=(), batch_count=1, cameras=2, n=7, width=W, height=H, device=torch.device("cpu"))
    assert outputs["hits"].shape == (2, 7) and outputs["hits"].dtype == torch.int32
    assert outputs["score"].shape == (2, 7) and outputs["score"].dtype == torch.float32
    # one entry per batch item, covering all cameras (one blend launch each)
    assert len(prepared) == 1 and prepared[0].key == (0, 1) and prepared[0].pixel_values.shape == (2, 2, H * W)
    with pytest.raises(ValueError, match="unique"):
        prepare_statistics([MaskedContributionCount("a", mask), MaskedContributionCount("a", mask)], batch_dims=(),
                           batch_count=1, cameras=1, n=1, width=W, height=H, device=torch.device("cpu"))
    with pytest.raises(ValueError, match="must use"):
        prepare_statistics([MaskedContributionCount("a", weights)], batch_dims=(), batch_count=1, cameras=1, n=1,
                           width=W, height=H, device=torch.device("cpu"))
    with pytest.raises(TypeError):
        prepare_statistics(["bogus"], batch_dims=(), batch_count=1, cameras=1, n=1, width=W, height=H,
                           device=torch.device("cpu"))


def test_pair_count_checks():
    # Totals beyond the int32 offsets are an overflow; view groups split at
    # the int32 limit, as the reference's per-view limit allows.
    from dsl_splat_amd.splatting import binning

    binning.check_pair_counts(0, 0)
    binning.check_pair_counts(binning.PAIR_LIMIT, binning.PAIR_LIMIT)
    with pytest.raises(OverflowError):
        binning.check_pair_counts(1, binning.PAIR_LIMIT + 1)
    limit = binning.PAIR_LIMIT
    assert binning.view_groups([limit // 2, limit // 2, 3]) == [(0, 2), (2, 3)]
    assert binning.view_groups([1, 2, 3]) == [(0, 3)]
    with pytest.raises(OverflowError):
        binning.view_groups([1, limit + 1])


def test_group_item_capacity_decays_after_a_large_frame():
    # The early-emission capacity of a binning shape follows the latest frame
    # with 12.5% headroom; after an unusually large frame it shrinks by 10% per
    # frame instead of staying at the largest frame's size.
    from types import SimpleNamespace

    from dsl_splat_amd.splatting import binning

    launch = SimpleNamespace(args=SimpleNamespace(tile_mode=0, n=10, views=1, width=16, height=16),
                             ranges=torch.empty(0))
    key = binning._shape_key(launch)
    saved = dict(binning._CAPACITY)
    binning._CAPACITY.clear()
    try:
        binning._remember_capacity(launch, 1000)
        assert binning._CAPACITY[key] == 1126
        binning._remember_capacity(launch, 100_000)
        assert binning._CAPACITY[key] == 112_501
        seen = []
        for _ in range(60):
            binning._remember_capacity(launch, 1000)
            seen.append(binning._CAPACITY[key])
        assert seen[0] == int(112_501 * 0.9)
        assert all(b <= a for a, b in zip(seen, seen[1:]))
        assert seen[-1] == 1126
    finally:
        binning._CAPACITY.clear()
        binning._CAPACITY.update(saved)


def test_depth_order_pass_count_and_key_bit_plan():
    # Passes of the depth order: bits 0-7, then 8-bit passes with the last
    # one widened to up to 10 bits, i.e. two passes up to 18 key bits, three
    # up to 26, four up to 32 (0 means 32; fewer than 9 bits still take two).
    from dsl_splat_amd.splatting import binning

    for bits in range(0, 33):
        end = 32 if bits == 0 else max(bits, 9)
        want = 2 if end <= 18 else 3 if end <= 26 else 4
        assert binning.order_pass_count(bits) == want, bits
    shape = ("test", 10, 1, 16, 16, "radius")
    saved = dict(binning._KEY_BITS)
    binning._KEY_BITS.clear()
    try:
        assert binning.planned_sort_bits(shape) == 0
        # First frame sorts all 32 bits: never a miss; the plan is its need.
        assert not binning.remember_key_bits(shape, 25, 0)
        assert binning.planned_sort_bits(shape) == 25
        # A smaller need in the same pass count keeps the plan.
        assert not binning.remember_key_bits(shape, 20, 25)
        assert binning.planned_sort_bits(shape) == 25
        # A larger need is a miss; the plan takes the most bits of its passes.
        assert binning.remember_key_bits(shape, 26, 25)
        assert binning.planned_sort_bits(shape) == 26
        assert binning.remember_key_bits(shape, 27, 26)
        assert binning.planned_sort_bits(shape) == 32
        # Fewer passes suffice again: the plan shrinks to the need.
        assert not binning.remember_key_bits(shape, 16, 32)
        assert binning.planned_sort_bits(shape) == 16
        # All kept keys equal (0 bits) still sort the two passes' 9 bits.
        assert not binning.remember_key_bits(shape, 0, 16)
        assert binning.order_pass_count(binning.planned_sort_bits(shape)) == 2
    finally:
        binning._KEY_BITS.clear()
        binning._KEY_BITS.update(saved)


def test_launch_wrappers_run_without_gradients():
    # native.no_grad turns gradients off inside the wrapped call (and only
    # there), also when the caller already has them off.
    from dsl_splat_amd.runtime import native

    seen = []

    @native.no_grad
    def probe(x):
        seen.append(torch.is_grad_enabled())
        return x * 2

    x = torch.ones(2, requires_grad=True)
    y = probe(x)
    assert seen == [False] and not y.requires_grad and torch.is_grad_enabled()
    with torch.no_grad():
        probe(x)
    assert seen == [False, False] and torch.is_grad_enabled()
    assert probe.__name__ == "probe"


def test_capped_list_stop_cache_keeps_recent_cameras(monkeypatch):
    # The stop cache (one int32 row per tile and camera) drops the least
    # recently rendered cameras beyond its byte limit; a camera rendered
    # again moves to the back, and its row is the latest frame's.
    from dsl_splat_amd.gs3d import lists as tile_lists

    tile_lists.clear()
    tiles = 1000
    monkeypatch.setattr(tile_lists, "CACHE_BYTES", 10 * tiles * 4)
    try:
        frames = []
        for f in range(6):
            stops = torch.full((2, tiles), f, dtype=torch.int32)
            lists = tile_lists.CappedLists([f * 2, f * 2 + 1], (None, 64, 48, "radius", 0), 7, None, stops, None)
            tile_lists.remember(lists)
            frames.append(stops)
        assert tile_lists._BYTES == 10 * tiles * 4
        shape = (None, 64, 48, "radius", 0)
        assert sorted(k[-1] for k in tile_lists._STOPS) == list(range(2, 12))
        again = torch.full((1, tiles), 99, dtype=torch.int32)
        tile_lists.remember(tile_lists.CappedLists([2], shape, 7, None, again, None))
        assert tile_lists._BYTES == 10 * tiles * 4
        assert next(reversed(tile_lists._STOPS))[-1] == 2
        stops, row, stream = tile_lists._STOPS[shape + (2,)]
        assert stops is again and row == 0 and stream == 7
        tile_lists.remember(tile_lists.CappedLists([100], shape, 7, None, again, None))
        assert shape + (3,) not in tile_lists._STOPS and shape + (2,) in tile_lists._STOPS
    finally:
        tile_lists.clear()
    assert tile_lists._BYTES == 0 and not tile_lists._STOPS


def test_capped_list_lengths_and_gate(monkeypatch):
    # capped_lengths keeps min(L, stop + stop/4 + 128) entries per tile (the
    # whole list for stop -1), the cap the id-write pass and the blend use;
    # frames below MIN_PAIRS tile pairs write whole lists.
    from dsl_splat_amd.gs3d import lists as tile_lists

    stops = torch.tensor([-1, 0, 7, 100, 4000, 4000], dtype=torch.int32)
    lengths = torch.tensor([50, 1000, 100, 10, 6000, 4999], dtype=torch.int32)
    want = [50, 128, 100, 10, 5128, 4999]
    assert tile_lists.capped_lengths(stops, lengths).tolist() == want
    # stop + stop/4 + 128 for the largest stop a list of 2^31 - 1 entries can report stays exact in int64
    big = torch.tensor([2**31 - 2], dtype=torch.int32)
    assert tile_lists.capped_lengths(big, torch.tensor([2**31 - 1], dtype=torch.int32)).tolist() == [2**31 - 1]
    monkeypatch.setattr(tile_lists, "ENABLED", True)
    assert tile_lists.applies(tile_lists.MIN_PAIRS, 1000)
    assert not tile_lists.applies(tile_lists.MIN_PAIRS - 1, 1000)
    assert not tile_lists.applies(tile_lists.MIN_PAIRS, 0)
    monkeypatch.setattr(tile_lists, "ENABLED", False)
    assert not tile_lists.applies(tile_lists.MIN_PAIRS, 1000)
