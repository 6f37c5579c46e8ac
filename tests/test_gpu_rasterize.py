"""End-to-end parity of the public entry points with the oracle pipeline.

gs3d.rasterize / gs3d.gsplat.rasterization / gs3d.ops run forward and
backward on the GPU for a loss sum(image * W) over every blended channel
(features, extra channels, alpha); the oracle composes the same stages on
the caller's quaternions.  Forward images and metadata are bit-exact; every
gradient entry is within rtol 1e-4 / atol 1e-5 of the oracle's, or, where
float32 summation order alone can move it further, within the entry's
stated float32 error bound (oracle_pipeline.check_gradient).
"""

import numpy as np
import pytest
import torch

import oracle
import oracle_pipeline
from oracle_pipeline import check_gradient, compare
from dsl_splat_amd import gs3d, synthetic
from dsl_splat_amd.cameras import PinholeCamera
from dsl_splat_amd.gs3d import gsplat, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


CASES = {
    "small_rgb_bg": dict(name="small", n=3000, width=96, height=80, seed=11, background=True),
    "sh3_4view": dict(name="sh3_1080p_4view", n=8000, width=160, height=96, seed=12),
    "sh3_720p_absgrad": dict(name="sh3_720p", n=6000, width=192, height=112, seed=13),
    "feat32_extra": dict(name="feat32", n=4000, width=128, height=96, seed=14),
    "pose_fanout": dict(name="pose_fanout", n=4000, width=160, height=96, seed=15),
}


def _run_case(key, entry="rasterize"):
    cfg = dict(CASES[key])
    name = cfg.pop("name")
    background = cfg.pop("background", False)
    scene = synthetic.make_scene(name, **cfg).to(DEV)
    print(f"case {key} entry={entry} views={scene.viewmats.shape[0]} n={len(scene.means)}", flush=True)
    return run_scene(scene, entry, background)


def run_scene(scene, entry="rasterize", background=False, oracle_threads=None):
    """Forward + backward of ``scene`` through a public entry point, compared
    with the oracle pipeline (bit-exact forward, gradient criterion); returns
    the forward outputs."""
    views = scene.viewmats.shape[0]
    params = dict(means=scene.means, quats=scene.quats, scales=scene.scales, opacities=scene.opacities)
    leaves = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    colors = (scene.sh_coeffs if scene.sh_coeffs is not None else scene.features).clone().requires_grad_(True)
    extra = None if scene.extra_features is None else scene.extra_features[0].clone().requires_grad_(True)
    viewmats = scene.viewmats.clone().requires_grad_(scene.pose_grad)
    bg = torch.rand((views, colors.shape[-1]), device=DEV) if background else None
    sh = scene.sh_coeffs is not None
    if entry == "rasterize":
        res = gs3d.rasterize(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"], viewmats,
                             scene.Ks, scene.width, scene.height, features=None if sh else colors,
                             sh_coeffs=colors if sh else None, sh_degree=scene.sh_degree, backgrounds=bg,
                             extra_features=extra, absgrad=scene.absgrad)
        feats, alpha, meta = res.features, res.alpha, res.meta
        ext = res.extra_features
    else:
        feats, alpha, meta = gsplat.rasterization(
            leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"], colors, viewmats, scene.Ks,
            scene.width, scene.height, near_plane=0.2, sh_degree=scene.sh_degree, packed=False, backgrounds=bg,
            absgrad=scene.absgrad, extra_signals=extra)
        ext = meta.get("render_extra_signals")
    W = scene.loss_weights
    D = feats.shape[-1]
    loss = (feats * W[..., :D]).sum() + (alpha * W[..., -1:]).sum()
    if ext is not None:
        loss = loss + (ext * W[..., D:-1]).sum()
    meta["means2d"].retain_grad()
    loss.backward()
    torch.cuda.synchronize()
    if oracle_threads:
        oracle.set_threads(oracle_threads)
    ref = oracle_pipeline.run(
        _np(scene.means), _np(scene.quats), _np(scene.scales), _np(scene.opacities), _np(scene.viewmats),
        _np(scene.Ks),
        scene.width, scene.height, features=None if sh else _np(colors), sh=_np(colors) if sh else None,
        sh_degree=scene.sh_degree, extra=None if extra is None else _np(extra),
        background=None if bg is None else _np(bg), upstream=_np(W), absgrad=scene.absgrad, normalize_quats=True,
        bounds=True)
    # Forward: bit-exact images and metadata.
    image = torch.cat([feats] + ([ext] if ext is not None else []) + [alpha], -1)
    np.testing.assert_array_equal(_np(image), ref["image"])
    proj = ref["proj"]
    np.testing.assert_array_equal(_np(meta["radii"])[..., 0], proj["radii"])
    np.testing.assert_array_equal(_np(meta["means2d"]), proj["means2d"])
    np.testing.assert_array_equal(_np(meta["conics"]), proj["meta_conics"])
    np.testing.assert_array_equal(_np(meta["opacities"]), proj["meta_opacities"])
    np.testing.assert_array_equal(_np(meta["tiles_per_gauss"]), proj["tiles"])
    assert meta["backend"] == "gs3d-hip" and meta["n_cameras"] == views
    # Backward: every entry within rtol 1e-4 / atol 1e-5 or its float32 bound.
    check_gradients(ref, leaves, colors, extra, meta, viewmats, scene, sh)
    return image, meta, ref


def check_gradients(ref, leaves, colors, extra, meta, viewmats, scene, sh):
    pg, rg, bd = ref["proj_grads"], ref["render_grads"], ref["bounds"]
    for name in ("means", "scales", "opacities", "quats"):
        check_gradient(name, _np(leaves[name].grad), pg[name], bd["proj"][name])
    if sh:
        check_gradient("sh_coeffs", _np(colors.grad), pg["sh"], bd["proj"]["sh"])
    else:
        check_gradient("features", _np(colors.grad), rg["features"], bd["render"]["features"])
    if extra is not None:
        check_gradient("extra", _np(extra.grad), rg["extra"], bd["render"]["extra"])
    check_gradient("means2d", _np(meta["means2d"].grad), rg["centers"], bd["render"]["centers"])
    if scene.absgrad:
        check_gradient("absgrad", _np(meta["means2d"].absgrad), rg["abs"], bd["render"]["abs"])
    if scene.pose_grad:
        check_gradient("viewmats", _np(viewmats.grad), ref["grad_viewmats"], bd["viewmats"])


@pytest.mark.parametrize("key", list(CASES))
def test_rasterize_matches_oracle(key):
    _run_case(key)


@pytest.mark.parametrize("key", ["sh3_720p_absgrad", "pose_fanout"])
def test_gsplat_adapter_matches_oracle(key):
    _run_case(key, entry="gsplat")


def test_gsplat_packed_metadata():
    scene = synthetic.make_scene("sh3_720p", n=3000, width=128, height=80, seed=21).to(DEV)
    means = scene.means.clone().requires_grad_(True)
    colors, alpha, meta = gsplat.rasterization(means, scene.quats, scene.scales, scene.opacities, scene.sh_coeffs,
                                               scene.viewmats, scene.Ks, scene.width, scene.height, sh_degree=3,
                                               absgrad=True)
    dense = gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks,
                           scene.width, scene.height, sh_coeffs=scene.sh_coeffs, near_plane=0.01, far_plane=1e10)
    visible = dense.meta["radii"][0, :, 0] > 0
    assert meta["packed"] and meta["gaussian_ids"].numel() == int(visible.sum())
    np.testing.assert_array_equal(_np(meta["gaussian_ids"]), np.nonzero(_np(visible))[0])
    np.testing.assert_array_equal(_np(meta["means2d"]), _np(dense.meta["means2d"][0][visible]))
    np.testing.assert_array_equal(_np(colors), _np(dense.features))
    (colors.sum() + alpha.sum()).backward()
    assert meta["means2d"].grad.shape == meta["means2d"].shape
    assert meta["means2d"].absgrad.shape == meta["means2d"].shape
    assert torch.all(meta["means2d"].absgrad >= meta["means2d"].grad.abs() - 1e-6)


def test_ops_staged_api_matches_fused():
    scene = synthetic.make_scene("small", n=3000, width=96, height=80, seed=31).to(DEV)
    cam = PinholeCamera(scene.viewmats[0], scene.Ks[0], scene.width, scene.height, near_plane=0.2,
                        far_plane=float("inf"))
    means = scene.means.clone().requires_grad_(True)
    feats = scene.features.clone().requires_grad_(True)
    geometry = ops.prepare_gaussians(means, scene.quats, scene.scales, scene.opacities, cam)
    tiles = ops.bin_and_sort(geometry)
    pix = ops.rasterize_to_pixels(geometry, tiles, feats)
    fused = gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks,
                           scene.width, scene.height, features=scene.features)
    np.testing.assert_array_equal(_np(pix.features), _np(fused.features[0]))
    np.testing.assert_array_equal(_np(pix.alpha), _np(fused.alpha[0]))
    W = scene.loss_weights[0]
    ((pix.features * W[..., :3]).sum() + (pix.alpha * W[..., 3:]).sum()).backward()
    m2 = scene.means.clone().requires_grad_(True)
    f2 = scene.features.clone().requires_grad_(True)
    r2 = gs3d.rasterize(m2, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, scene.width,
                        scene.height, features=f2)
    ((r2.features[0] * W[..., :3]).sum() + (r2.alpha[0] * W[..., 3:]).sum()).backward()
    compare("ops_means", _np(means.grad), _np(m2.grad), rtol=1e-4, atol=1e-5 * float(m2.grad.abs().max()))
    compare("ops_features", _np(feats.grad), _np(f2.grad), rtol=1e-4, atol=1e-6)


def test_empty_and_culled_inputs():
    scene = synthetic.make_scene("small", n=500, width=64, height=48, seed=41).to(DEV)
    # Everything behind the camera: no pairs, background only, zero gradients.
    means = (-scene.means).clone().requires_grad_(True)
    bg = torch.tensor([[0.2, 0.4, 0.6]], device=DEV)
    res = gs3d.rasterize(means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, 64, 48,
                         features=scene.features, backgrounds=bg)
    assert torch.all(res.meta["radii"] == 0)
    assert torch.equal(res.features[0], bg[0].expand(48, 64, 3))
    assert torch.all(res.alpha == 0)
    res.features.sum().backward()
    assert torch.all(means.grad == 0)
    # N = 0.
    empty = torch.zeros((0, 3), device=DEV)
    res0 = gs3d.rasterize(empty, torch.zeros((0, 4), device=DEV), empty, torch.zeros((0,), device=DEV),
                          scene.viewmats, scene.Ks, 64, 48, features=torch.zeros((0, 3), device=DEV))
    assert res0.features.shape == (1, 48, 64, 3) and torch.all(res0.alpha == 0)


@pytest.mark.parametrize("cameras,bad", [(1, 0), (3, 2), (4, 1)])
def test_camera_errors_raise(cameras, bad):
    # The status codes of every camera travel with the pair totals in one
    # read-back; an error on any camera (odd and even counts) must surface.
    scene = synthetic.make_scene("small", n=100, width=32, height=32, seed=51).to(DEV)
    rows = torch.arange(cameras, device=DEV) % scene.viewmats.shape[0]
    viewmats, Ks = scene.viewmats[rows].contiguous(), scene.Ks[rows].contiguous()
    K = Ks.clone()
    K[bad, 0, 1] = 0.1
    with pytest.raises(NotImplementedError):
        gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, viewmats, K, 32, 32,
                       features=scene.features)
    K = Ks.clone()
    K[bad, 0, 0] = float("nan")
    with pytest.raises(ValueError):
        gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, viewmats, K, 32, 32,
                       features=scene.features)
    # Valid cameras still render after the failures.
    res = gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, viewmats, Ks, 32, 32,
                         features=scene.features)
    assert res.features.shape[0] == cameras and torch.isfinite(res.features).all()
    V = viewmats.clone()
    V[bad, 2] = V[bad, 1]
    sh = torch.zeros((100, 4, 3), device=DEV)
    with pytest.raises(torch.linalg.LinAlgError):
        gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, V, Ks, 32, 32, sh_coeffs=sh)


def _leaf(t):
    return t.detach().clone().requires_grad_(True)


def test_batched_inputs_match_per_item_calls():
    # Leading batch dimensions (B=2, 4 cameras each): every batch item renders
    # exactly as a separate call on that item, gradients included.
    a = synthetic.make_scene("sh3_1080p_4view", n=3000, width=128, height=80, seed=61).to(DEV)
    b = synthetic.make_scene("sh3_1080p_4view", n=3000, width=128, height=80, seed=62).to(DEV)
    print("batched inputs B=2 C=4", flush=True)
    stack = lambda name: torch.stack([getattr(a, name), getattr(b, name)])
    params = {k: _leaf(stack(k)) for k in ("means", "quats", "scales", "opacities", "sh_coeffs")}
    viewmats, Ks = stack("viewmats"), stack("Ks")
    W = torch.stack([a.loss_weights, b.loss_weights])
    res = gs3d.rasterize(params["means"], params["quats"], params["scales"], params["opacities"], viewmats, Ks,
                         a.width, a.height, sh_coeffs=params["sh_coeffs"], sh_degree=3)
    assert res.features.shape == (2, 4, a.height, a.width, 3) and res.alpha.shape == (2, 4, a.height, a.width, 1)
    ((res.features * W[..., :3]).sum() + (res.alpha * W[..., 3:]).sum()).backward()
    for i in range(2):
        item = {k: _leaf(v[i]) for k, v in params.items()}
        one = gs3d.rasterize(item["means"], item["quats"], item["scales"], item["opacities"], viewmats[i], Ks[i],
                             a.width, a.height, sh_coeffs=item["sh_coeffs"], sh_degree=3)
        np.testing.assert_array_equal(_np(res.features[i]), _np(one.features))
        np.testing.assert_array_equal(_np(res.alpha[i]), _np(one.alpha))
        np.testing.assert_array_equal(_np(res.meta["radii"][i]), _np(one.meta["radii"]))
        np.testing.assert_array_equal(_np(res.meta["means2d"][i]), _np(one.meta["means2d"]))
        ((one.features * W[i, ..., :3]).sum() + (one.alpha * W[i, ..., 3:]).sum()).backward()
        for k in item:
            g = _np(item[k].grad)
            compare(f"batch{i}_{k}", _np(params[k].grad[i]), g, rtol=1e-4, atol=1e-5 * max(1.0, float(np.abs(g).max())))


def test_packed_metadata_several_cameras_and_batches():
    # Packed metadata over (batch, camera, Gaussian): the triples with both
    # radii positive in row-major order, their values and index vectors, and
    # means2d.grad / absgrad equal to the dense gradients at those entries.
    a = synthetic.make_scene("sh3_1080p_4view", n=2500, width=128, height=80, seed=71).to(DEV)
    b = synthetic.make_scene("sh3_1080p_4view", n=2500, width=128, height=80, seed=72).to(DEV)
    print("packed metadata B=2 C=4", flush=True)
    stack = lambda name: torch.stack([getattr(a, name), getattr(b, name)])
    args = [stack(k) for k in ("means", "quats", "scales", "opacities")]
    viewmats, Ks, sh = stack("viewmats"), stack("Ks"), stack("sh_coeffs")
    W = torch.stack([a.loss_weights, b.loss_weights])
    out = {}
    for packed in (False, True):
        res = gs3d.rasterize(*[_leaf(t) for t in args], viewmats, Ks, a.width, a.height, sh_coeffs=sh, sh_degree=3,
                             packed=packed, absgrad=True)
        ((res.features * W[..., :3]).sum() + (res.alpha * W[..., 3:]).sum()).backward()
        out[packed] = res
    dense, packed = out[False].meta, out[True].meta
    visible = (dense["radii"] > 0).all(-1)  # (B, C, N)
    bi, ci, gi = (_np(t) for t in visible.nonzero(as_tuple=True))
    assert packed["packed"] and not dense["packed"]
    np.testing.assert_array_equal(_np(packed["batch_ids"]), bi)
    np.testing.assert_array_equal(_np(packed["camera_ids"]), ci)
    np.testing.assert_array_equal(_np(packed["gaussian_ids"]), gi)
    for name in ("radii", "means2d", "opacities", "conics", "tiles_per_gauss"):
        np.testing.assert_array_equal(_np(packed[name]), _np(dense[name])[bi, ci, gi])
    np.testing.assert_array_equal(_np(out[True].features), _np(out[False].features))
    for attr in ("grad", "absgrad"):
        want = _np(getattr(dense["means2d"], attr))[bi, ci, gi]
        compare(f"packed_means2d_{attr}", _np(getattr(packed["means2d"], attr)), want, rtol=1e-4,
                atol=1e-5 * max(1.0, float(np.abs(want).max())))


@pytest.mark.parametrize("during_forward", [True, False])
def test_repeated_backward_and_interleaved_frames(monkeypatch, during_forward):
    # The blend VJP accumulates into buffers that the forward blend launch
    # clears (or, with GS3D_CLEAR_IN_BACKWARD, the backward): a second
    # backward of the same graph (retain_graph) must use fresh buffers
    # (gradients add up to twice one backward), and two frames whose
    # forwards run before either backward must keep their own buffers.
    from dsl_splat_amd.gs3d import autograd

    monkeypatch.setattr(autograd, "CLEAR_DURING_FORWARD", during_forward)
    scene = synthetic.make_scene("sh3_720p", n=4000, width=128, height=96, seed=17).to(DEV)
    print("repeated backward, interleaved frames", flush=True)
    W = scene.loss_weights

    def frame(leaves, sh, absgrad):
        res = gs3d.rasterize(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
                             scene.viewmats, scene.Ks, scene.width, scene.height, sh_coeffs=sh, sh_degree=3,
                             absgrad=absgrad)
        return (res.features * W[..., :3]).sum() + (res.alpha * W[..., 3:]).sum()

    def close(got, want):
        # Run-to-run differences come only from the order of float atomics.
        torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-6 * float(want.abs().max().clamp(min=1.0)))

    def fresh():
        leaves = {k: getattr(scene, k).clone().requires_grad_(True) for k in ("means", "quats", "scales", "opacities")}
        return leaves, scene.sh_coeffs.clone().requires_grad_(True)

    for absgrad in (False, True):
        leaves, sh = fresh()
        frame(leaves, sh, absgrad).backward()
        once = {k: v.grad.clone() for k, v in leaves.items()} | {"sh": sh.grad.clone()}
        leaves, sh = fresh()
        loss = frame(leaves, sh, absgrad)
        loss.backward(retain_graph=True)
        loss.backward()
        for k, v in list(leaves.items()) + [("sh", sh)]:
            close(v.grad, 2 * once[k])
        # Two forwards, then both backwards in reverse order.
        la, sa = fresh()
        lb, sb = fresh()
        loss_a = frame(la, sa, absgrad)
        loss_b = frame(lb, sb, absgrad)
        loss_b.backward()
        loss_a.backward()
        for k in leaves:
            close(la[k].grad, once[k])
            close(lb[k].grad, once[k])
        close(sa.grad, once["sh"])
    # A forward that needs gradients but is never differentiated.
    leaves, sh = fresh()
    frame(leaves, sh, False)
    torch.cuda.synchronize()


def test_clearing_in_backward_matches_clearing_during_forward(monkeypatch):
    # With GS3D_CLEAR_IN_BACKWARD the blend VJP's accumulation buffers are
    # allocated and zeroed by the backward instead of by the forward blend
    # launch: the same gradients (atomic order aside).
    from dsl_splat_amd.gs3d import autograd

    scene = synthetic.make_scene("sh3_1080p_4view", n=8000, width=288, height=240, seed=21).to(DEV)
    print("clearing in backward vs during forward", flush=True)
    grads = []
    for during_forward in (True, False):
        monkeypatch.setattr(autograd, "CLEAR_DURING_FORWARD", during_forward)
        means = scene.means.clone().requires_grad_(True)
        sh = scene.sh_coeffs.clone().requires_grad_(True)
        res = gs3d.rasterize(means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks,
                             scene.width, scene.height, sh_coeffs=sh, sh_degree=3, absgrad=True)
        W = scene.loss_weights
        ((res.features * W[..., :3]).sum() + (res.alpha * W[..., 3:]).sum()).backward()
        grads.append((means.grad.cpu(), sh.grad.cpu(), res.meta["means2d"].absgrad.cpu()))
    for a, b in zip(*grads):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6)
