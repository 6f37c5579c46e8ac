"""Capped tile lists (dsl_splat_amd/gs3d/lists.py).

The id-write pass given caps writes each tile's first min(L, cap) entries
and nothing else; gs3d_bin_redo then completes exactly the flagged tiles.
Rasterization with caps, whether the caps are the last frame's stops of
the same cameras, forced far too small or random, gives the images of whole
lists bit for bit and the same gradients (float atomic order aside), and
reports a stop per tile that covers every pixel's contributors.
"""

import dataclasses

import numpy as np
import pytest
import torch

from dsl_splat_amd import gs3d, synthetic
from dsl_splat_amd.gs3d import api
from dsl_splat_amd.gs3d import lists as tile_lists
from dsl_splat_amd.gs3d import projection as gproj
from dsl_splat_amd.gs3d import render as grender
from dsl_splat_amd.splatting import binning, cameras

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _say(*args):
    print(*args, flush=True)


def _cap(stops):
    """Entries a list keeps under each stop (int64; -1: all)."""
    stops = stops.astype(np.int64)
    return np.where(stops < 0, np.iinfo(np.int64).max, stops + stops // 4 + 128)


def _dense(name, n, width, height, seed, scale=1.0, views=None, opacity=None):
    """A synthetic scene with its Gaussians ``scale`` times larger and, with
    ``opacity``, opacities uniform in [opacity, 0.99] (dense enough that many
    tiles terminate before their lists end)."""
    scene = synthetic.make_scene(name, n=n, width=width, height=height, seed=seed)
    scene.scales = scene.scales * scale
    if opacity is not None:
        g = torch.Generator().manual_seed(seed)
        scene.opacities = opacity + (0.99 - opacity) * torch.rand(n, generator=g)
    if views is not None and views != scene.viewmats.shape[0]:
        reps = -(-views // scene.viewmats.shape[0])
        scene = dataclasses.replace(scene, viewmats=scene.viewmats.repeat(reps, 1, 1)[:views],
                                    Ks=scene.Ks.repeat(reps, 1, 1)[:views], loss_weights=None)
    return scene.to(DEV)


def _project(scene, degree):
    quats = torch.nn.functional.normalize(scene.quats, dim=-1)
    with_centers = bool(degree)
    full, _, centers, _ = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height, with_centers)
    return gproj.project_views(
        scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks, scene.width,
        scene.height, 0.2, float("inf"), 0.0, sh=scene.sh_coeffs if degree is not None else None,
        sh_degree=degree or 0, camera_centers=centers if with_centers else None, metadata=True)


def _capped_items(ranges, ids, depths, caps, width, height):
    """Group items the capped id-write pass must read, from the whole lists.

    A group's items are the rows that touch any of its 8x8 tiles (radius
    mode: a row's tile square meets the group exactly where it covers
    tiles), in depth order (ties by row).  The pass reads, per group, every
    512-item chunk that starts at or before the item holding some tile's
    min(L, cap)-th entry; returns that count and the group item total."""
    V, N = depths.shape
    gx, gy = (width + 15) // 16, (height + 15) // 16
    sgx, sgy = (gx + 7) // 8, (gy + 7) // 8
    tpv, gpv = gx * gy, sgx * sgy
    T = V * tpv
    lengths = ranges[:, 1] - ranges[:, 0]
    t = np.arange(T)
    local = t % tpv
    group = (t // tpv) * gpv + (local // gx // 8) * sgx + (local % gx) // 8
    # depth rank of every (view, row), ties by row
    rank = np.empty(V * N, np.int64)
    for v in range(V):
        o = np.lexsort((np.arange(N), depths[v]))
        rank[v * N + o] = np.arange(N)
    tile_of = np.repeat(t, lengths)
    key = group[tile_of].astype(np.int64) * (V * N) + rank[(tile_of // tpv) * N + ids]
    items = np.unique(key)
    item_group = items // (V * N)
    group_start = np.searchsorted(item_group, np.arange(V * gpv))
    pos = np.searchsorted(items, key) - group_start[group[tile_of]]
    k = np.minimum(lengths, caps)
    need = np.zeros(V * gpv, np.int64)
    has = k > 0
    last_pos = pos[(ranges[:, 0] + k - 1)[has]]
    np.maximum.at(need, group[has], last_pos // 512 + 1)
    size = np.bincount(item_group, minlength=V * gpv)
    return int(np.minimum(need * 512, size).sum()), len(items)


class _PoisonedTorch:
    """torch, except that new int32 tensors start filled with -1 (so an id
    the write pass should have written and did not shows up)."""

    def __getattr__(self, name):
        return getattr(torch, name)

    @staticmethod
    def empty(*size, dtype=None, **kw):
        t = torch.empty(*size, dtype=dtype, **kw)
        if dtype == torch.int32:
            t.fill_(-1)
        return t


WRITE_CASES = {
    # name, n, width, height, seed, scale, views, SH degree, tile mode, early emission
    "sh3_radius": ("sh3_1080p_4view", 40000, 160, 96, 31, 1.0, None, 3, "radius", False),
    "sh3_radius_early": ("sh3_1080p_4view", 40000, 160, 96, 32, 1.0, None, 3, "radius", True),
    "rgb_snugbox": ("small", 30000, 96, 80, 33, 1.0, None, None, "snugbox", False),
    "rgb_accutile": ("small", 30000, 96, 80, 34, 1.0, None, None, "accutile", False),
    # Eight 1080p cameras: more than 1024 tile groups, so the group items
    # take the multi-pass sort and the redo pass reads them from the other
    # half of the scratch.
    "groups_multipass": ("sh3_1080p_4view", 40000, 1920, 1080, 35, 2.0, 8, 0, "radius", False),
}


@pytest.mark.parametrize("key", list(WRITE_CASES))
def test_capped_write_pass_writes_each_tile_prefix(key, monkeypatch):
    name, n, W, H, seed, scale, views, degree, mode, early = WRITE_CASES[key]
    scene = _dense(name, n, W, H, seed, scale, views)
    _say(f"capped write pass {key}: views={scene.viewmats.shape[0]} n={n} {W}x{H} {mode}")
    st = _project(scene, degree)
    order, offsets, totals = binning.order_rows(st.centers, st.radii, st.depths, W, H, conics=st.conics,
                                                tile_mode=mode)
    S, M = totals.cpu().tolist()
    ref_ranges, ref_ids = binning.bin_rows(st.centers, st.radii, order, offsets, S, M, W, H, conics=st.conics,
                                           tile_mode=mode)
    ranges_np = _np(ref_ranges).astype(np.int64)
    lengths = ranges_np[:, 1] - ranges_np[:, 0]
    tiles = len(lengths)
    rng = np.random.default_rng(seed)
    stops = rng.integers(-1, max(int(lengths.max()), 2), size=tiles).astype(np.int32)
    stops[rng.random(tiles) < 0.3] = 0
    keep_len = np.minimum(lengths, _cap(stops))
    assert (keep_len < lengths).sum() > tiles // 10, "too few tiles capped for the case to test anything"
    monkeypatch.setattr(binning, "torch", _PoisonedTorch())
    launch = binning.prepare_bin_rows(st.centers, st.radii, order, offsets, W, H, conics=st.conics, tile_mode=mode)
    got_early = None
    if early:
        shape = binning._shape_key(launch)
        binning._CAPACITY[shape] = S + 1000
        try:
            got_early = binning.emit_early(launch)
        finally:
            binning._CAPACITY.pop(shape, None)
        assert got_early is not None
    caps = torch.from_numpy(stops).to(DEV)
    redo_list = torch.full((tiles + 1,), 77, dtype=torch.int32, device=DEV)
    ranges, ids = binning.launch_bin_rows(launch, S, M, got_early, caps=caps, redo_list=redo_list)
    assert launch.scratch is not None
    assert int(redo_list[0]) == 0 and bool((redo_list[1:] == 77).all())  # the count only
    np.testing.assert_array_equal(_np(ranges), _np(ref_ranges))
    tile_of = np.repeat(np.arange(tiles), lengths)
    pos = np.arange(M) - np.repeat(ranges_np[:, 0], lengths)
    want = _np(ref_ids)

    def check(written):
        got = _np(ids)
        np.testing.assert_array_equal(got[written], want[written])
        assert (got[~written] == -1).all(), "ids written beyond a tile's cap"

    check(pos < keep_len[tile_of])
    # The items the capped pass read: every chunk (kChunk = 512 consecutive
    # items of a group) that some tile of the group still needed, i.e. that
    # starts before the tile's min(L, cap)-th entry.  With every cap at
    # infinity that is every item.
    loaded = binning.capped_items_loaded(launch)
    assert 0 < loaded <= S
    if mode == "radius":
        want_loaded, group_items = _capped_items(ranges_np, want, _np(st.depths), _cap(stops), W, H)
        assert group_items == S
        assert loaded == want_loaded
    flags = (rng.random(tiles) < 0.3).astype(np.int32)
    listed = np.concatenate([[flags.sum()], np.flatnonzero(flags), np.zeros(tiles - flags.sum())]).astype(np.int32)
    flags_t, listed_t = torch.from_numpy(flags).to(DEV), torch.from_numpy(listed).to(DEV)
    # A redo pass whose list counts no tile writes nothing, whatever the flags.
    none = listed_t.clone()
    none[0] = 0
    binning.native.call("gs3d_bin_redo", binning.ctypes.byref(launch.args), binning.native.ptr(flags_t),
                        binning.native.ptr(none), binning.native.ptr(launch.scratch), launch.scratch.numel(),
                        binning.native.stream(torch.device(DEV)))
    check(pos < keep_len[tile_of])
    binning.redo_bin_rows(launch, flags_t, listed_t)
    assert launch.scratch is None
    check((pos < keep_len[tile_of]) | (flags[tile_of] != 0))


def test_blend_stops_cover_every_contributor():
    scene = _dense("sh3_1080p_4view", 40000, 160, 96, 36, scale=2.0, opacity=0.6)
    W, H = scene.width, scene.height
    _say("blend stops against contributors")
    st = _project(scene, 3)
    order, offsets, totals = binning.order_rows(st.centers, st.radii, st.depths, W, H, conics=st.conics)
    S, M = totals.cpu().tolist()
    ranges, ids = binning.bin_rows(st.centers, st.radii, order, offsets, S, M, W, H, conics=st.conics)
    views = st.centers.shape[0]
    tiles = ranges.shape[0]
    stops = torch.full((views, tiles // views), -7, dtype=torch.int32, device=DEV)
    lists = tile_lists.CappedLists([], (), 0, None, stops, None)
    out = grender.render_views(ranges, ids, st.centers, st.conics, st.colors, W, H, lists=lists)
    ref = grender.render_views(ranges, ids, st.centers, st.conics, st.colors, W, H)
    for a, b in ((out.features, ref.features), (out.alpha, ref.alpha), (out.contributors, ref.contributors)):
        assert torch.equal(a, b)
    gx, gy = (W + 15) // 16, (H + 15) // 16
    contrib = _np(ref.contributors)
    padded = np.zeros((views, gy * 16, gx * 16), np.int64)
    padded[:, :H, :W] = contrib
    most = padded.reshape(views, gy, 16, gx, 16).max(axis=(2, 4)).reshape(-1)
    s = _np(stops).reshape(-1).astype(np.int64)
    r = _np(ranges).astype(np.int64)
    lengths = r[:, 1] - r[:, 0]
    assert ((s == -1) | ((s >= 0) & (s <= lengths))).all()
    assert (most[s >= 0] <= s[s >= 0]).all()
    assert (s >= 0).sum() > len(s) // 5, "many tiles of a dense scene terminate"
    assert (s[s >= 0] + s[s >= 0] // 4 + 128 < lengths[s >= 0]).sum() > len(s) // 10, "and long before their ends"


def _image_and_grads(scene, features=None, extra=None, viewmats=None, tile_mode="radius", background=None):
    leaves = {k: getattr(scene, k).clone().requires_grad_(True) for k in ("means", "quats", "scales", "opacities")}
    sh = scene.sh_coeffs is not None
    colors = (scene.sh_coeffs if sh else features).clone().requires_grad_(True)
    ext = None if extra is None else extra.clone().requires_grad_(True)
    res = gs3d.rasterize(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
                         scene.viewmats if viewmats is None else viewmats, scene.Ks, scene.width, scene.height,
                         features=None if sh else colors, sh_coeffs=colors if sh else None,
                         sh_degree=scene.sh_degree if sh else None, extra_features=ext, tile_mode=tile_mode,
                         backgrounds=background, absgrad=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    loss = (res.features * torch.rand(res.features.shape, generator=g, device=DEV)).sum() + res.alpha.sum()
    if res.extra_features is not None:
        loss = loss + (res.extra_features * torch.rand(res.extra_features.shape, generator=g, device=DEV)).sum()
    loss.backward()
    images = [res.features, res.alpha] + ([res.extra_features] if res.extra_features is not None else [])
    grads = [v.grad for v in leaves.values()] + [colors.grad, res.meta["means2d"].absgrad]
    if ext is not None:
        grads.append(ext.grad)
    return [t.detach().clone() for t in images], [t.clone() for t in grads]


def _same(got, want):
    for a, b in zip(got[0], want[0]):
        assert torch.equal(a, b)
    for a, b in zip(got[1], want[1]):
        # Run-to-run differences come only from the order of float atomics.
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6 * float(b.abs().max().clamp(min=1.0)))


E2E_CASES = {
    "sh3_4view": dict(name="sh3_1080p_4view", n=40000, width=160, height=96, seed=41),
    "rgb_background_snugbox": dict(name="small", n=30000, width=96, height=80, seed=42, tile_mode="snugbox",
                                   background=True),
    "rgb_accutile": dict(name="small", n=30000, width=96, height=80, seed=43, tile_mode="accutile"),
    # 80 feature channels + 3 extra + alpha: two channel windows.
    "two_windows": dict(name="small", n=30000, width=96, height=80, seed=44, channels=80, extra=3),
}
DENSE = dict(scale=2.0, opacity=0.6)


@pytest.mark.parametrize("key", list(E2E_CASES))
def test_capped_lists_match_whole_lists(key, monkeypatch):
    cfg = dict(E2E_CASES[key])
    tile_mode = cfg.pop("tile_mode", "radius")
    channels = cfg.pop("channels", None)
    extra_ch = cfg.pop("extra", None)
    background = cfg.pop("background", False)
    scene = _dense(cfg.pop("name"), cfg["n"], cfg["width"], cfg["height"], cfg["seed"], **DENSE)
    views = scene.viewmats.shape[0]
    g = torch.Generator().manual_seed(cfg["seed"])
    features = scene.features
    if channels is not None:
        features = torch.rand((cfg["n"], channels), generator=g).to(DEV)
    extra = torch.rand((cfg["n"], extra_ch), generator=g).to(DEV) if extra_ch else None
    bg = torch.rand((views, features.shape[-1] if features is not None else 3), generator=g).to(DEV) \
        if background else None
    run = lambda: _image_and_grads(scene, features, extra, tile_mode=tile_mode, background=bg)  # noqa: E731
    seen = []
    real_remember = tile_lists.remember
    monkeypatch.setattr(tile_lists, "remember", lambda lists: (seen.append(lists), real_remember(lists))[1])
    monkeypatch.setattr(tile_lists, "MIN_PAIRS", 0)
    ranges = []
    real_bin = api.launch_bin_rows
    monkeypatch.setattr(api, "launch_bin_rows", lambda *a, **k: (lambda r: (ranges.append(r[0]), r)[1])(
        real_bin(*a, **k)))
    tile_lists.clear()
    try:
        _say(f"capped lists {key}: whole lists")
        monkeypatch.setattr(tile_lists, "ENABLED", False)
        want = run()
        assert not seen
        monkeypatch.setattr(tile_lists, "ENABLED", True)
        _say(f"capped lists {key}: first frame (stops measured)")
        _same(run(), want)
        first = seen[-1]
        assert first.caps is None
        _say(f"capped lists {key}: caps from the last frame")
        _same(run(), want)
        steady = seen[-1]
        assert steady.caps is not None and int(steady.redo.sum()) == 0
        assert torch.equal(steady.stops, first.stops)
        # The case caps lists: some tile's cap lies before its list's end.
        r = _np(ranges[-1]).astype(np.int64)
        assert (_cap(_np(steady.caps)) < r[:, 1] - r[:, 0]).any()
        _say(f"capped lists {key}: caps far too small")
        for t, i, _ in tile_lists._STOPS.values():
            t[i].fill_(0)
        _same(run(), want)
        forced = seen[-1]
        flagged = int(forced.redo.sum())
        assert flagged > 0
        listed = _np(forced.redo_list)
        assert listed[0] == flagged
        assert sorted(listed[1:1 + flagged].tolist()) == np.flatnonzero(_np(forced.redo)).tolist()
        _say(f"capped lists {key}: random caps")
        rng = torch.Generator(device=DEV).manual_seed(7)
        for t, i, _ in tile_lists._STOPS.values():
            t[i].copy_(torch.randint(-1, 400, t[i].shape, generator=rng, device=DEV, dtype=torch.int32))
        _same(run(), want)
    finally:
        tile_lists.clear()


def test_capped_lists_follow_the_cameras(monkeypatch):
    # Stops are keyed by camera: the same cameras in another order, and a
    # frame with cameras seen and unseen, find their own rows.
    scene = _dense("sh3_1080p_4view", 40000, 160, 96, 45, **DENSE)
    seen = []
    real_remember = tile_lists.remember
    monkeypatch.setattr(tile_lists, "remember", lambda lists: (seen.append(lists), real_remember(lists))[1])
    monkeypatch.setattr(tile_lists, "MIN_PAIRS", 0)
    tile_lists.clear()
    try:
        perm = torch.tensor([3, 1, 0, 2], device=DEV)
        rotated = scene.viewmats[perm]
        monkeypatch.setattr(tile_lists, "ENABLED", False)
        want_perm = _image_and_grads(dataclasses.replace(scene, Ks=scene.Ks[perm]), viewmats=rotated)
        monkeypatch.setattr(tile_lists, "ENABLED", True)
        _say("capped lists: four cameras, then the same four in another order")
        _image_and_grads(scene)
        base = seen[-1]
        _same(_image_and_grads(dataclasses.replace(scene, Ks=scene.Ks[perm]), viewmats=rotated), want_perm)
        moved = seen[-1]
        assert moved.caps is not None and int(moved.redo.sum()) == 0
        assert torch.equal(moved.stops, base.stops[perm])
        assert torch.equal(moved.caps.view_as(moved.stops), base.stops[perm])
        _say("capped lists: two known cameras and two new ones")
        two = dataclasses.replace(scene, Ks=scene.Ks[:2].clone(), viewmats=scene.viewmats[:2].clone())
        tile_lists.clear()
        _image_and_grads(two)
        mixed_views = scene.viewmats.clone()
        mixed_views[2:, :3, 3] += 0.25  # two cameras moved: new keys
        monkeypatch.setattr(tile_lists, "ENABLED", False)
        want_mixed = _image_and_grads(scene, viewmats=mixed_views)
        monkeypatch.setattr(tile_lists, "ENABLED", True)
        _same(_image_and_grads(scene, viewmats=mixed_views), want_mixed)
        mixed = seen[-1]
        caps = mixed.caps.view_as(mixed.stops)
        assert torch.equal(caps[:2], seen[-2].stops)
        assert bool((caps[2:] == -1).all())
    finally:
        tile_lists.clear()


def test_camera_keys():
    scene = _dense("sh3_1080p_4view", 100, 160, 96, 46)
    views = torch.cat([scene.viewmats, scene.viewmats[:1]])
    Ks = torch.cat([scene.Ks, scene.Ks[:1]])
    views[4, 0, 0] = torch.nextafter(views[4, 0, 0], torch.tensor(2.0, device=DEV))  # one ulp: the same key
    keys = torch.empty(5, dtype=torch.int64, device=DEV)
    cameras.launch_prepare(views, Ks, scene.width, scene.height, False, keys=keys)
    k = keys.tolist()
    assert len(set(k[:4])) == 4
    assert k[4] == k[0]
    moved = views.clone()
    moved[:, 2, 3] += 0.5
    keys2 = torch.empty(5, dtype=torch.int64, device=DEV)
    cameras.launch_prepare(moved, Ks, scene.width, scene.height, False, keys=keys2)
    assert not set(keys2.tolist()) & set(k)
    zero = torch.eye(4, device=DEV)[None].clone()
    negzero = zero.clone()
    negzero[0, 0, 1] = -0.0
    kz = torch.empty(2, dtype=torch.int64, device=DEV)
    cameras.launch_prepare(torch.cat([zero, negzero]), Ks[:1].repeat(2, 1, 1), scene.width, scene.height, False,
                           keys=kz)
    assert kz[0] == kz[1]


def test_batch_items_sharing_cameras_keep_their_own_stops(monkeypatch):
    # Two batch items render different Gaussians through the same cameras:
    # each finds its own stops on the next call (no overflow), and the images
    # equal those of whole lists.
    a = _dense("sh3_1080p_4view", 40000, 160, 96, 47, **DENSE)
    b = _dense("sh3_1080p_4view", 40000, 160, 96, 48, **DENSE)
    stack = lambda name: torch.stack([getattr(a, name), getattr(b, name)])  # noqa: E731
    args = [stack(k) for k in ("means", "quats", "scales", "opacities")]
    viewmats = torch.stack([a.viewmats, a.viewmats])
    Ks = torch.stack([a.Ks, a.Ks])
    sh = stack("sh_coeffs")
    seen = []
    real_remember = tile_lists.remember
    monkeypatch.setattr(tile_lists, "remember", lambda lists: (seen.append(lists), real_remember(lists))[1])
    monkeypatch.setattr(tile_lists, "MIN_PAIRS", 0)
    tile_lists.clear()
    try:
        run = lambda: gs3d.rasterize(*args, viewmats, Ks, a.width, a.height, sh_coeffs=sh,  # noqa: E731
                                     sh_degree=3)
        monkeypatch.setattr(tile_lists, "ENABLED", False)
        want = run()
        monkeypatch.setattr(tile_lists, "ENABLED", True)
        _say("batched items sharing cameras: first call, then one with caps")
        run()
        first = seen[-2:]
        got = run()
        second = seen[-2:]
        for i in range(2):
            assert second[i].caps is not None and int(second[i].redo.sum()) == 0
            assert torch.equal(second[i].caps.view_as(second[i].stops), first[i].stops)
        assert not torch.equal(first[0].stops, first[1].stops)
        assert torch.equal(got.features, want.features) and torch.equal(got.alpha, want.alpha)
    finally:
        tile_lists.clear()


def test_capped_lists_on_empty_and_partly_empty_frames(monkeypatch):
    # With caps on for every frame size: a frame whose Gaussians are all
    # behind the cameras (no tile pairs), then one where only one camera sees
    # any, each rendered twice (the second time with the first's stops), equal
    # the same frames rendered with whole lists.
    scene = _dense("sh3_1080p_4view", 20000, 160, 96, 49, **DENSE)
    monkeypatch.setattr(tile_lists, "MIN_PAIRS", 0)
    hidden = scene.means.clone()
    hidden[:, 2] = -1000.0
    views = scene.viewmats.clone()
    views[1:, :3, 3] += torch.tensor([0.0, 0.0, 1000.0], device=DEV)  # cameras 1-3 far beyond everything
    cases = {"all culled": (hidden, scene.viewmats), "three cameras empty": (scene.means, views)}
    tile_lists.clear()
    try:
        for name, (means, vm) in cases.items():
            _say(f"capped lists, {name}")
            run = lambda: gs3d.rasterize(means, scene.quats, scene.scales, scene.opacities, vm, scene.Ks,  # noqa
                                         scene.width, scene.height, sh_coeffs=scene.sh_coeffs, sh_degree=3)
            monkeypatch.setattr(tile_lists, "ENABLED", False)
            want = run()
            monkeypatch.setattr(tile_lists, "ENABLED", True)
            for _ in range(2):
                got = run()
                assert torch.equal(got.features, want.features) and torch.equal(got.alpha, want.alpha)
            torch.cuda.synchronize()
    finally:
        tile_lists.clear()
