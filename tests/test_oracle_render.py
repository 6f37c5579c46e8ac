"""Pins for the oracle's blending forward/backward (gs3d/render.py:36-356)
against the independent float64 Torch renderer and closed forms."""

import numpy as np
import torch

import torch_ref
from dsl_splat_amd import synthetic


def _pipeline(oracle_lib, scene, features=None, background=None, extra=None, tile_mode="radius"):
    full, inverse, cent, err = oracle_lib.camera_prepare(scene.viewmats.numpy(), scene.Ks.numpy(),
                                                         scene.width, scene.height, False)
    out = oracle_lib.project_fwd(scene.means.numpy(), scene.quats.numpy(), scene.scales.numpy(),
                                 scene.opacities.numpy(), scene.viewmats.numpy(), full, scene.Ks.numpy(),
                                 scene.width, scene.height, tile_mode=tile_mode)
    offsets, total = oracle_lib.scan_i32(out["tiles"].ravel())
    keys, vals = oracle_lib.emit_keys(out["centers"], out["radii"], out["depths"], offsets, total,
                                      scene.width, scene.height, conics=out["conics"], tile_mode=tile_mode)
    views = scene.viewmats.shape[0]
    T = views * ((scene.width + 15) // 16) * ((scene.height + 15) // 16)
    sk, sv = oracle_lib.sort_pairs(keys, vals, 32 + int(T).bit_length())
    ranges = oracle_lib.tile_ranges(sk, T)
    feats = scene.features.numpy() if features is None else features
    image, final_t, contrib = oracle_lib.render_fwd(scene.width, scene.height, ranges, sv, out["centers"],
                                                    out["conics"], feats, extra=extra, background=background)
    return out, ranges, sv, image, final_t, contrib


def _torch_order(out, v=0):
    vis = np.nonzero(out["radii"][v] > 0)[0]
    bits = out["depths"][v][vis].view(np.uint32)
    return vis[np.lexsort((vis, bits))]


def test_render_forward_matches_float64(oracle_lib):
    scene = synthetic.make_scene("small", n=80, width=48, height=40, seed=2)
    bg = np.array([[0.1, 0.2, 0.3]], np.float32)
    out, ranges, ids, image, final_t, contrib = _pipeline(oracle_lib, scene, background=bg)
    c = torch.tensor(out["centers"][0], dtype=torch.float64)
    k = torch.tensor(out["conics"][0], dtype=torch.float64)
    ref, T = torch_ref.render(c, k[:, :3], k[:, 3], scene.features.double(), _torch_order(out), 48, 40,
                              background=torch.tensor(bg[0], dtype=torch.float64),
                              radii=torch.tensor(out["radii"][0]))
    np.testing.assert_allclose(image[0], ref.numpy(), atol=1e-5, rtol=1e-4)
    np.testing.assert_allclose(final_t[0], T.numpy(), atol=1e-6, rtol=1e-4)
    # Alpha channel = 1 - T_final (both are sums of the same weights).
    np.testing.assert_allclose(image[0, ..., -1], 1.0 - final_t[0], atol=2e-6)
    assert contrib.max() > 0


def test_render_empty_tiles_and_single_gaussian(oracle_lib):
    # One Gaussian at a pixel centre: alpha there equals min(0.99, opacity)
    # exactly (exp(0) = 1), tiles it does not touch show the background.
    W = H = 64
    centers = np.array([[[20.0, 20.0]]], np.float32)
    conics = np.array([[[0.05, 0.0, 0.05, 0.6]]], np.float32)
    feats = np.array([[0.25, 0.5, 1.0]], np.float32)
    gx = 4
    ranges = np.zeros((16, 2), np.int32)
    ids = np.zeros(4, np.int32)
    for t, (tx, ty) in enumerate([(0, 0), (1, 0), (0, 1), (1, 1)]):
        ranges[ty * gx + tx] = [t, t + 1]
    bg = np.array([[0.5, 0.5, 0.5]], np.float32)
    image, final_t, contrib = oracle_lib.render_fwd(W, H, ranges, ids, centers, conics, feats, background=bg)
    # (the background term is fused: one rounding, so within one ulp)
    np.testing.assert_allclose(image[0, 20, 20, :3], 0.6 * feats[0].astype(np.float64) + 0.4 * bg[0], rtol=1.2e-7)
    assert image[0, 20, 20, 3] == np.float32(0.6)
    assert final_t[0, 20, 20] == np.float32(1.0) - np.float32(0.6)
    np.testing.assert_array_equal(image[0, 50, 50], [0.5, 0.5, 0.5, 0.0])
    assert final_t[0, 50, 50] == 1.0 and contrib[0, 50, 50] == 0
    assert contrib[0, 20, 20] == 1


def test_render_termination_rule(oracle_lib):
    # Opaque stack at one pixel: the blend stops before the Gaussian that
    # would push T below 1e-4 (gs3d/render.py:98-100), without blending it.
    W = H = 16
    k = 6
    centers = np.tile(np.array([[[8.0, 8.0]]], np.float32), (1, k, 1))
    conics = np.tile(np.array([[[0.5, 0.0, 0.5, 0.95]]], np.float32), (1, k, 1))
    feats = np.eye(k, 3, dtype=np.float32) + 0.01
    ranges = np.array([[0, k]], np.int32)
    ids = np.arange(k, dtype=np.int32)
    image, final_t, contrib = oracle_lib.render_fwd(W, H, ranges, ids, centers, conics, feats)
    # T: 0.05, 0.0025, 1.25e-4 (>= 1e-4, blends), then 6.25e-6 < 1e-4 stops:
    # three Gaussians blend and the fourth is not blended.
    assert contrib[0, 8, 8] == 3
    np.testing.assert_allclose(final_t[0, 8, 8], 0.05 ** 3, rtol=1e-5)


def test_render_backward_matches_autograd(oracle_lib):
    scene = synthetic.make_scene("small", n=60, width=40, height=36, seed=4)
    bg = np.array([[0.3, 0.1, 0.2]], np.float32)
    out, ranges, ids, image, final_t, contrib = _pipeline(oracle_lib, scene, background=bg)
    rng = np.random.default_rng(0)
    up = rng.normal(size=image.shape).astype(np.float32)
    grads = oracle_lib.render_bwd(40, 36, ranges, ids, out["centers"], out["conics"], scene.features.numpy(),
                                  final_t, contrib, up, background=bg, absgrad=True)
    c = torch.tensor(out["centers"][0], dtype=torch.float64, requires_grad=True)
    k = torch.tensor(out["conics"][0, :, :3], dtype=torch.float64, requires_grad=True)
    o = torch.tensor(out["conics"][0, :, 3], dtype=torch.float64, requires_grad=True)
    f = scene.features.double().requires_grad_(True)
    ref, _ = torch_ref.render(c, k, o, f, _torch_order(out), 40, 36, background=torch.tensor(bg[0]).double(),
                              radii=torch.tensor(out["radii"][0]))
    (ref * torch.tensor(up[0], dtype=torch.float64)).sum().backward()
    vis = out["radii"][0] > 0
    scale = lambda a: 1e-4 * np.abs(a).max()
    np.testing.assert_allclose(grads["centers"][0][vis], c.grad.numpy()[vis], rtol=2e-3, atol=scale(c.grad.numpy()))
    np.testing.assert_allclose(grads["conics"][0][vis, :3], k.grad.numpy()[vis], rtol=2e-3, atol=scale(k.grad.numpy()))
    np.testing.assert_allclose(grads["conics"][0][vis, 3], o.grad.numpy()[vis], rtol=2e-3, atol=scale(o.grad.numpy()))
    np.testing.assert_allclose(grads["features"][vis], f.grad.numpy()[vis], rtol=2e-3, atol=scale(f.grad.numpy()))
    # |per-pixel| sums dominate the signed sums.
    assert np.all(grads["abs"][0] >= np.abs(grads["centers"][0]) - 1e-6)
