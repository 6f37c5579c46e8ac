"""Pins for the oracle's projection (gs3d/projection.py:89-164) and its VJP
(gs3d/projection.py:198-285) against independent statements."""

import math

import numpy as np
import torch

import torch_ref
from dsl_splat_amd import synthetic


def _camera(scene, oracle_lib, with_centers=False):
    full, inverse, centers, err = oracle_lib.camera_prepare(
        scene.viewmats.numpy(), scene.Ks.numpy(), scene.width, scene.height, with_centers)
    assert np.all(err == 0)
    return full, inverse, centers


def _project(scene, oracle_lib, **kw):
    full, _, _ = _camera(scene, oracle_lib)
    out = oracle_lib.project_fwd(scene.means.numpy(), scene.quats.numpy(), scene.scales.numpy(),
                                 scene.opacities.numpy(), scene.viewmats.numpy(), full, scene.Ks.numpy(),
                                 scene.width, scene.height, **kw)
    return out, full


def test_projection_matches_float64_ewa(oracle_lib):
    scene = synthetic.make_scene("small", n=3000, seed=1)
    out, _ = _project(scene, oracle_lib)
    vis = out["radii"][0] > 0
    assert vis.mean() > 0.9
    c64, k64, o64, z64, cov = torch_ref.project(
        scene.means.double(), scene.quats.double(), scene.scales.double(), scene.opacities.double(),
        scene.viewmats[0].double(), scene.Ks[0].double(), scene.width, scene.height)
    np.testing.assert_allclose(out["centers"][0][vis], c64.numpy()[vis], atol=2e-4, rtol=1e-6)
    np.testing.assert_allclose(out["conics"][0][vis, :3], k64.detach().numpy()[vis], rtol=2e-4, atol=1e-4)
    np.testing.assert_array_equal(out["conics"][0][vis, 3], scene.opacities.numpy()[vis])
    np.testing.assert_allclose(out["depths"][0][vis], z64.numpy()[vis], rtol=1e-6)
    # Radius = ceil(3 sqrt(lambda_max)); away from integer boundaries the
    # float32 restatement must agree with the float64 value exactly.
    covn = cov.detach().numpy()
    checked = 0
    for i in np.nonzero(vis)[0][:2000]:
        r = torch_ref.radius_of(covn[i])
        if abs(r - round(r)) > 1e-3:
            assert out["radii"][0][i] == math.ceil(r), (i, r, out["radii"][0][i])
            checked += 1
    assert checked > 1000
    # Tile count equals the clamped rectangle area (CUDA getRect).
    for i in np.nonzero(vis)[0][:500]:
        x0, y0, x1, y1 = torch_ref.rect_tiles(out["centers"][0][i], out["radii"][0][i], scene.width, scene.height)
        assert out["tiles"][0][i] == (x1 - x0) * (y1 - y0)
    # Culled rows: zero radii/tiles and zeroed geometry.
    assert np.all(out["tiles"][0][~vis] == 0)
    assert np.all(out["centers"][0][~vis] == 0)


def test_projection_special_cases(oracle_lib):
    # Isotropic Gaussian with identity rotation straight ahead of an identity
    # camera: cov2 = s^2 f^2/z^2 I + 0.3, centre = (cx-0.5, cy-0.5).
    W = H = 64
    f, z, s = 100.0, 5.0, 0.05
    means = np.array([[0.0, 0.0, z]], np.float32)
    quats = np.array([[1.0, 0.0, 0.0, 0.0]], np.float32)
    scales = np.full((1, 3), s, np.float32)
    K = np.array([[[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]]], np.float32)
    V = np.eye(4, dtype=np.float32)[None]
    full, _, _, _ = oracle_lib.camera_prepare(V, K, W, H, False)
    out = oracle_lib.project_fwd(means, quats, scales, np.array([0.7], np.float32), V, full, K, W, H)
    var = (s * f / z) ** 2 + 0.3
    np.testing.assert_allclose(out["conics"][0, 0, :3], [1 / var, 0.0, 1 / var], rtol=1e-5, atol=1e-7)
    assert out["radii"][0, 0] == math.ceil(3 * math.sqrt(var))
    np.testing.assert_allclose(out["centers"][0, 0], [W / 2 - 0.5, H / 2 - 0.5], atol=1e-5)
    assert out["depths"][0, 0] == np.float32(z)
    # Near/far/radius-clip culling.
    for kw in (dict(near_plane=5.0), dict(far_plane=5.0), dict(radius_clip=float(out["radii"][0, 0]))):
        o2 = oracle_lib.project_fwd(means, quats, scales, np.array([0.7], np.float32), V, full, K, W, H, **kw)
        assert o2["radii"][0, 0] == 0 and o2["tiles"][0, 0] == 0
    # Behind the camera.
    o3 = oracle_lib.project_fwd(-means, quats, scales, np.array([0.7], np.float32), V, full, K, W, H)
    assert o3["radii"][0, 0] == 0
    # Entirely off-screen: rectangle clamps to zero area.
    o4 = oracle_lib.project_fwd(np.array([[100.0, 0.0, z]], np.float32), quats, scales,
                                np.array([0.7], np.float32), V, full, K, W, H)
    assert o4["radii"][0, 0] == 0 and o4["tiles"][0, 0] == 0


def _random_gaussian(rng, saturate=False):
    mean = rng.normal(scale=0.4, size=3)
    mean[2] = 4.0 + rng.random()
    if saturate:
        mean[0] = 12.0  # x/z far beyond 1.3 * W / (2 fx)
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    s = np.exp(rng.uniform(-3.0, -1.5, size=3))
    return mean, q, s, float(rng.uniform(0.2, 0.9))


def _cam(rng, W=320, H=240):
    V = np.eye(4)
    a = rng.normal(scale=0.1, size=3)
    Rm = torch_ref.quat_to_rot(torch.tensor(np.r_[1.0, a] / np.linalg.norm(np.r_[1.0, a]))).numpy()
    V[:3, :3] = Rm
    V[:3, 3] = rng.normal(scale=0.2, size=3)
    fx, fy = 300.0, 280.0
    K = np.array([[fx, 0, W / 2 + 3], [0, fy, H / 2 - 2], [0, 0, 1]])
    px, py = 2 * fx / W, 2 * fy / H
    cx, cy = 2 * K[0, 2] / W - 1, 2 * K[1, 2] / H - 1
    P = np.stack([px * V[0] + cx * V[2], py * V[1] + cy * V[2], V[2], V[2]])
    return V, P, K, W, H


def test_projection_vjp_matches_central_differences(oracle_lib):
    # Exact-derivative pieces: float64 VJP vs central differences of the
    # float64 projection loss (unsaturated clamp; the 1e-7 regulariser only
    # shifts the inverse-covariance VJP by det^2/(det^2+1e-7) ~ 1 - 1e-6).
    rng = np.random.default_rng(7)
    for _ in range(25):
        mean, q, s, o = _random_gaussian(rng)
        V, P, K, W, H = _cam(rng)
        gc, gk = rng.normal(size=2), rng.normal(size=4)
        args = lambda m, qq, ss, oo, VV, PP: oracle_lib.projection_loss_f64(
            m, qq, ss, oo, VV, PP, W, H, K[0, 0], K[1, 1], gc, gk)
        vjp = oracle_lib.projection_vjp_f64(mean, q, s, o, V, P, W, H, K[0, 0], K[1, 1], gc, gk)

        def fd(vec, idx, build):
            h = 1e-6 * max(1.0, abs(vec[idx]))
            p, m = vec.copy(), vec.copy()
            p[idx] += h
            m[idx] -= h
            return (build(p) - build(m)) / (2 * h)

        for i in range(3):
            assert abs(fd(mean, i, lambda x: args(x, q, s, o, V, P)) - vjp["mean"][i]) < 2e-4 * (1 + abs(vjp["mean"][i]))
            assert abs(fd(s, i, lambda x: args(mean, q, x, o, V, P)) - vjp["scale"][i]) < 2e-4 * (1 + abs(vjp["scale"][i]))
        for i in range(4):
            assert abs(fd(q, i, lambda x: args(mean, x, s, o, V, P)) - vjp["quat"][i]) < 2e-4 * (1 + abs(vjp["quat"][i]))
        assert abs(fd(np.array([o]), 0, lambda x: args(mean, q, s, x[0], V, P)) - vjp["opacity"]) < 1e-6
        Vf, Pf = V.ravel(), P.ravel()
        for i in range(16):
            gv = fd(Vf, i, lambda x: args(mean, q, s, o, x.reshape(4, 4), P))
            gp = fd(Pf, i, lambda x: args(mean, q, s, o, V, x.reshape(4, 4)))
            assert abs(gv - vjp["view"].ravel()[i]) < 2e-4 * (1 + abs(gv)), (i, gv, vjp["view"].ravel()[i])
            assert abs(gp - vjp["proj"].ravel()[i]) < 2e-4 * (1 + abs(gp)), (i, gp, vjp["proj"].ravel()[i])


def test_projection_vjp_custom_adjoints(oracle_lib):
    # Known answers for the two conventions that are not exact derivatives:
    # a saturated clamp component is a constant (splatting/geometry.py:42-51)
    # and the inverse covariance uses 1/(det^2+1e-7) (geometry.py:61-71).
    # The independent float64 autograd statement in torch_ref encodes both.
    rng = np.random.default_rng(8)
    for saturate in (False, True):
        for _ in range(10):
            mean, q, s, o = _random_gaussian(rng, saturate=saturate)
            V, P, K, W, H = _cam(rng)
            gc, gk = rng.normal(size=2), rng.normal(size=4)
            vjp = oracle_lib.projection_vjp_f64(mean, q, s, o, V, P, W, H, K[0, 0], K[1, 1], gc, gk)
            m = torch.tensor(mean[None], requires_grad=True)
            qq = torch.tensor(q[None], requires_grad=True)
            ss = torch.tensor(s[None], requires_grad=True)
            VV = torch.tensor(V, requires_grad=True)
            centers, conic, _, _, _ = torch_ref.project(m, qq, ss, torch.tensor([o]), VV, torch.tensor(K), W, H)
            loss = (centers[0] * torch.tensor(gc)).sum() + (conic[0] * torch.tensor(gk[:3])).sum()
            loss.backward()
            np.testing.assert_allclose(vjp["scale"], ss.grad[0].numpy(), rtol=1e-6, atol=1e-9)
            np.testing.assert_allclose(vjp["quat"], qq.grad[0].numpy(), rtol=1e-6, atol=1e-9)
            # The torch statement differentiates the centre through K and V
            # directly; the oracle through P (then the camera VJP maps P to
            # V).  Means see both paths identically.
            np.testing.assert_allclose(vjp["mean"], m.grad[0].numpy(), rtol=1e-5, atol=1e-8)
            P_grad_to_V = _projection_grad_to_view(vjp["proj"], K, W, H)
            np.testing.assert_allclose(vjp["view"] + P_grad_to_V, VV.grad.numpy(), rtol=1e-5, atol=1e-7)


def _projection_grad_to_view(gP, K, W, H):
    px, py = 2 * K[0, 0] / W, 2 * K[1, 1] / H
    cx, cy = 2 * K[0, 2] / W - 1, 2 * K[1, 2] / H - 1
    g = np.zeros((4, 4))
    g[0] = px * gP[0]
    g[1] = py * gP[1]
    g[2] = cx * gP[0] + cy * gP[1] + gP[2] + gP[3]
    return g


def test_float32_vjp_tracks_float64(oracle_lib):
    # The float32 oracle VJP (used as the GPU checker) against its float64
    # instantiation, one Gaussian at a time.
    scene = synthetic.make_scene("small", n=200, seed=3)
    out, full = _project(scene, oracle_lib)
    rng = np.random.default_rng(9)
    gc = rng.normal(size=(1, 200, 2)).astype(np.float32)
    gk = rng.normal(size=(1, 200, 4)).astype(np.float32)
    g32 = oracle_lib.project_bwd(scene.means.numpy(), scene.quats.numpy(), scene.scales.numpy(),
                                 scene.opacities.numpy(), scene.viewmats.numpy(), full, scene.Ks.numpy(),
                                 scene.width, scene.height, out["radii"], gc, gk)
    K = scene.Ks[0].numpy()
    view64 = np.zeros((4, 4))
    proj64 = np.zeros((4, 4))
    for i in range(200):
        if out["radii"][0, i] <= 0:
            assert np.all(g32["means"][i] == 0)
            continue
        v = oracle_lib.projection_vjp_f64(scene.means[i].numpy(), scene.quats[i].numpy(), scene.scales[i].numpy(),
                                          float(scene.opacities[i]), scene.viewmats[0].numpy(), full[0],
                                          scene.width, scene.height, K[0, 0], K[1, 1], gc[0, i], gk[0, i])
        view64 += v["view"]
        proj64 += v["proj"]
        for name, key in (("means", "mean"), ("quats", "quat"), ("scales", "scale")):
            np.testing.assert_allclose(g32[name][i], v[key], rtol=2e-3, atol=2e-3 * np.abs(v[key]).max() + 1e-6)
    np.testing.assert_allclose(g32["view"][0], view64, rtol=2e-3, atol=1e-3 * np.abs(view64).max())
    np.testing.assert_allclose(g32["projection"][0], proj64, rtol=2e-3, atol=1e-3 * np.abs(proj64).max())


def test_quaternion_normalization_matches_torch(oracle_lib):
    # The projection normalises raw quaternions as torch.nn.functional.normalize
    # (reference inputs.py:252) and differentiates through it; checked against
    # torch float64 autograd, with the zero and tiny quaternions clamped at 1e-12.
    g = torch.Generator().manual_seed(4)
    q = torch.randn((500, 4), generator=g) * torch.rand((500, 1), generator=g) * 10
    q[0] = 0.0
    q[1] = torch.tensor([1.0, 0.0, 0.0, 0.0])
    q[2] = 3e-13
    up = torch.randn((500, 4), generator=g)
    u, grad = oracle_lib.normalize_quats(q.numpy(), up.numpy())
    q64 = q.double().requires_grad_(True)
    ref = torch.nn.functional.normalize(q64, dim=-1)
    ref.backward(up.double())
    np.testing.assert_allclose(u, ref.detach().numpy(), rtol=2e-7, atol=1e-7)
    big = np.abs(q.numpy()).max(-1) > 1e-6
    np.testing.assert_allclose(grad[big], q64.grad.numpy()[big], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(u[0], np.zeros(4, np.float32))
    np.testing.assert_array_equal(u[1], [1.0, 0.0, 0.0, 0.0])
    np.testing.assert_allclose(grad[0], up[0].numpy() / np.float32(1e-12), rtol=1e-6)
